// Non-causal flash attention forward for gfx950 (bf16 MFMA, fp32 softmax).
//
// Replaces the reference's splash kernel: kernels/splash.py:566-650
// (`attention`), its body _flash_attention_kernel :115-375 (online update
// :250-267, kv_len masking :216-218/:277-331, normalize :369-375) and the
// residual form :665-742.
//
// Two kernels:
//   * flash_fwd_d128_kernel (D = 128, every DiT workload) in
//     flash_fwd_d128.hip;
//   * flash_fwd_kernel (generic, used for D = 64), described here.
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

#include <mutex>

#include "../../include/dt_attention.h"
#include "dt_common.h"
#include "flash_common.h"

namespace dt {

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
  const int kv_end = resolve_len(p.kv_len_dev, p.kv_end, p.Skv);

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
      if (it < C::K_ITEMS && kv < kv_end)
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
        if (it < C::V_ITEMS && kv < kv_end)
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

  const int ntiles = (kv_end + C::BKV - 1) / C::BKV;
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
    if (kv0 + C::BKV > kv_end) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int kv = kv0 + kb * 32 + 8 * (r >> 2) + 4 * hf + (r & 3);
          if (kv >= kv_end)
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


template <int D, int NW, int QB>
static int launch(const FlashParams& base, hipStream_t st) {
  using C = FlashCfg<D, NW, QB>;
  FlashParams p = base;
  p.n_qblk = (p.Sq + C::BQ - 1) / C::BQ;
  const int64_t nwg = (int64_t)p.n_qblk * p.Hq * p.B;
  if (nwg > 0x7fffffff)
    return set_error(DT_ERR_SHAPE, "dt_flash_fwd: grid too large");
  p.n_wg = (int)nwg;
  static std::atomic<uint64_t> lds_set{0};
  if (int rc = ensure_lds_limit((const void*)flash_fwd_kernel<D, NW, QB>,
                                C::LDS_BYTES, lds_set, "dt_flash_fwd"))
    return rc;
  hipLaunchKernelGGL((flash_fwd_kernel<D, NW, QB>), dim3(p.n_wg),
                     dim3(C::NT), C::LDS_BYTES, st, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return set_error(DT_ERR_LAUNCH, "dt_flash_fwd: %s", hipGetErrorString(e));
  return DT_OK;
}

static bool al16(const void* ptr) { return ((uintptr_t)ptr & 15u) == 0; }

}  // namespace dt

namespace dt {
namespace {

// Validation and dispatch shared by dt_flash_fwd (bf16 keys) and
// dt_flash_fwd_qk8 (E4M3 keys, k_e4m3).
int flash_entry(const uint16_t* q, const void* k, bool k_e4m3,
                const uint16_t* v, uint16_t* o, int B, int Hq, int Hkv, int Sq,
                int Skv, int D, const int64_t* q_strides,
                const int64_t* k_strides, const int64_t* v_strides,
                const int64_t* o_strides, float scale, int kv_len,
                const float* mk, const int32_t* tile_span,
                const int32_t* tile_ids, float* o32, float* m, float* l,
                void* stream, const uint16_t* vt = nullptr,
                int64_t vt_tiles = 0, void* ws = nullptr, size_t ws_bytes = 0,
                const int32_t* kv_len_dev = nullptr) {
  const bool resid = (o32 != nullptr) || (m != nullptr) || (l != nullptr);
  const bool packed = vt != nullptr;
  if (!q || !k || !q_strides || !k_strides ||
      (!packed && (!v || !v_strides)))
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
  // With the length in device memory the host plans for every key: the
  // grid, the packed-V tile count and the split cover Skv, and the kernels
  // skip the tiles past the length they read.
  if (kv_len_dev != nullptr) kv_len = 0;
  if (k_e4m3 && D != 128)
    return set_error(DT_ERR_UNSUPPORTED,
                     "dt_flash_fwd_qk8: head dim %d (supported: 128)", D);
  if ((tile_span != nullptr) != (tile_ids != nullptr))
    return set_error(DT_ERR_ARG,
                     "dt_flash_fwd_blocksparse: tile_span and tile_ids must "
                     "both be given");
  if (packed) {
    if (D != 128)
      return set_error(DT_ERR_UNSUPPORTED,
                       "dt_flash_fwd_ex: packed V needs head dim 128, got %d", D);
    const int kv_end = (kv_len <= 0) ? Skv : kv_len;
    const int64_t need = (int64_t)(kv_end + 63) / 64;
    if (vt_tiles < need)
      return set_error(DT_ERR_SHAPE,
                       "dt_flash_fwd_ex: vt_tiles %lld < %lld key tiles",
                       (long long)vt_tiles, (long long)need);
    if (!al16(vt))
      return set_error(DT_ERR_UNSUPPORTED,
                       "dt_flash_fwd_ex: misaligned packed V");
  }
  if (tile_span && D != 128)
    return set_error(DT_ERR_UNSUPPORTED,
                     "dt_flash_fwd_blocksparse: head dim %d (supported: 128)",
                     D);
  for (int i = 0; i < 3; ++i) {
    if (q_strides[i] % 8 || k_strides[i] % (k_e4m3 ? 16 : 8) ||
        (!packed && v_strides[i] % 8) || (o && o_strides[i] % 4))
      return set_error(DT_ERR_UNSUPPORTED,
                       "dt_flash_fwd: strides must be multiples of 8 elements "
                       "(16 for E4M3 keys)");
  }
  if (!al16(q) || !al16(k) || (!packed && !al16(v)) || (o && ((uintptr_t)o & 7u)) ||
      (o32 && !al16(o32)))
    return set_error(DT_ERR_UNSUPPORTED, "dt_flash_fwd: misaligned tensor");
  FlashParams p;
  p.q = q;
  p.k = k_e4m3 ? nullptr : (const uint16_t*)k;
  p.k8 = k_e4m3 ? (const uint8_t*)k : nullptr;
  p.tile_span = tile_span;
  p.tile_ids = tile_ids;
  p.v = packed ? nullptr : v;
  p.vt = vt;
  p.vt_tiles = vt_tiles;
  p.o = o;
  p.o32 = o32;
  p.m = m;
  p.l = l;
  p.mk = mk;
  p.kv_len_dev = kv_len_dev;
  p.q_sb = q_strides[0];
  p.q_sh = q_strides[1];
  p.q_ss = q_strides[2];
  p.k_sb = k_strides[0];
  p.k_sh = k_strides[1];
  p.k_ss = k_strides[2];
  p.v_sb = packed ? 0 : v_strides[0];
  p.v_sh = packed ? 0 : v_strides[1];
  p.v_ss = packed ? 0 : v_strides[2];
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
  p.ws = nullptr;
  p.n_split = 1;
  p.n_tail = 0;
  p.n_main = 0;
  if (D == 128 && ws != nullptr) {
    if (!al16(ws))
      return set_error(DT_ERR_UNSUPPORTED, "dt_flash_fwd_ex: misaligned workspace");
    int n_cu = 0;
    if (int rc = device_cu_count(&n_cu)) return rc;
    const int64_t n_wg = (int64_t)B * Hq * ((Sq + 255) / 256);
    const SplitPlan sp =
        split_plan(n_wg, (p.kv_end + 63) / 64, n_cu, ws_bytes);
    if (sp.n_split > 1 && sp.ws_bytes <= ws_bytes) {
      p.ws = (float*)ws;
      p.n_split = sp.n_split;
      p.n_tail = sp.n_tail;
      p.n_main = sp.n_main;
    }
  }
  if (D == 128) return launch_flash_d128(p, st);
  return launch<64, 4, 1>(p, st);
}

}  // namespace
}  // namespace dt

extern "C" int dt_flash_fwd(const uint16_t* q, const uint16_t* k,
                            const uint16_t* v, uint16_t* o, int B, int Hq,
                            int Hkv, int Sq, int Skv, int D,
                            const int64_t* q_strides, const int64_t* k_strides,
                            const int64_t* v_strides, const int64_t* o_strides,
                            float scale, int kv_len, const float* mk,
                            float* o32, float* m, float* l, void* stream) {
  return dt::flash_entry(q, k, false, v, o, B, Hq, Hkv, Sq, Skv, D, q_strides,
                         k_strides, v_strides, o_strides, scale, kv_len, mk,
                         nullptr, nullptr, o32, m, l, stream);
}

extern "C" int dt_flash_fwd_qk8(const uint16_t* q, const uint8_t* k8,
                                const uint16_t* v, uint16_t* o, int B, int Hq,
                                int Hkv, int Sq, int Skv, int D,
                                const int64_t* q_strides,
                                const int64_t* k_strides,
                                const int64_t* v_strides,
                                const int64_t* o_strides, float scale,
                                int kv_len, const float* mk, float* o32,
                                float* m, float* l, void* stream) {
  return dt::flash_entry(q, k8, true, v, o, B, Hq, Hkv, Sq, Skv, D, q_strides,
                         k_strides, v_strides, o_strides, scale, kv_len, mk,
                         nullptr, nullptr, o32, m, l, stream);
}

extern "C" int dt_flash_fwd_blocksparse(
    const uint16_t* q, const void* k, int k_format, const uint16_t* v,
    uint16_t* o, int B, int Hq, int Hkv, int Sq, int Skv, int D,
    const int64_t* q_strides, const int64_t* k_strides,
    const int64_t* v_strides, const int64_t* o_strides, float scale,
    int kv_len, const float* mk, const int32_t* tile_span,
    const int32_t* tile_ids, float* o32, float* m, float* l, void* stream) {
  if (k_format != 0 && k_format != 1)
    return dt::set_error(DT_ERR_ARG,
                         "dt_flash_fwd_blocksparse: k_format %d (0 bf16, 1 "
                         "E4M3)", k_format);
  if (!tile_span || !tile_ids)
    return dt::set_error(DT_ERR_ARG,
                         "dt_flash_fwd_blocksparse: null tile table");
  return dt::flash_entry(q, k, k_format == 1, v, o, B, Hq, Hkv, Sq, Skv, D,
                         q_strides, k_strides, v_strides, o_strides, scale,
                         kv_len, mk, tile_span, tile_ids, o32, m, l, stream);
}

extern "C" size_t dt_flash_fwd_workspace_bytes(int B, int Hq, int Sq, int Skv,
                                               int kv_len, int D) {
  if (D != 128 || B <= 0 || Hq <= 0 || Sq <= 0 || Skv <= 0) return 0;
  int n_cu = 0;
  if (dt::device_cu_count(&n_cu) != DT_OK) return 0;
  const int kv_end = (kv_len <= 0 || kv_len > Skv) ? Skv : kv_len;
  const int64_t n_wg = (int64_t)B * Hq * ((Sq + 255) / 256);
  return dt::split_plan(n_wg, (kv_end + 63) / 64, n_cu).ws_bytes;
}

// ---- dt_flash_fwd_ex_noalloc: the split workspace in static device memory.
//
// `scratch` is a file-scope device array (one copy per GPU, allocated when
// the library's code object loads on that GPU and held until the process
// ends).  Host code never uses the array's name as an address: it is a
// host-side stand-in.  The device address comes from hipGetSymbolAddress,
// taken once per device with that device current and kept in
// g_scratch_dev[]; only that pointer reaches the kernels.
static __device__ __align__(256) uint8_t scratch[DT_NOALLOC_SCRATCH_BYTES];

namespace dt {
namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_dev[kMaxDevices];

// the current device's address of `scratch` (looked up on first use)
int scratch_address(void** out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess)
    return set_error(DT_ERR_LAUNCH, "dt_flash_fwd_ex_noalloc: no current device");
  if (dev < 0 || dev >= kMaxDevices)
    return set_error(DT_ERR_UNSUPPORTED,
                     "dt_flash_fwd_ex_noalloc: device %d >= %d", dev,
                     kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_dev[dev] == nullptr) {
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || ptr == nullptr)
      return set_error(DT_ERR_LAUNCH,
                       "dt_flash_fwd_ex_noalloc: scratch address: %s",
                       hipGetErrorString(e));
    g_scratch_dev[dev] = ptr;
  }
  *out = g_scratch_dev[dev];
  return DT_OK;
}

}  // namespace
}  // namespace dt

extern "C" int dt_flash_fwd_ex_noalloc(
    const uint16_t* q, const void* k, int k_format, const uint16_t* v,
    const int64_t* v_strides, const uint16_t* vt, int64_t vt_tiles, uint16_t* o,
    int B, int Hq, int Hkv, int Sq, int Skv, int D, const int64_t* q_strides,
    const int64_t* k_strides, const int64_t* o_strides, float scale,
    int kv_len, const int32_t* kv_len_dev, const float* mk,
    const int32_t* tile_span, const int32_t* tile_ids, float* o32, float* m,
    float* l, size_t scratch_bytes, void* stream) {
  if (scratch_bytes > (size_t)DT_NOALLOC_SCRATCH_BYTES)
    return dt::set_error(DT_ERR_ARG,
                         "dt_flash_fwd_ex_noalloc: scratch_bytes %zu above the "
                         "static scratch of %zu bytes",
                         scratch_bytes, (size_t)DT_NOALLOC_SCRATCH_BYTES);
  void* ws = nullptr;
  if (scratch_bytes > 0)
    if (int rc = dt::scratch_address(&ws)) return rc;
  return dt_flash_fwd_ex(q, k, k_format, v, v_strides, vt, vt_tiles, o, B, Hq,
                         Hkv, Sq, Skv, D, q_strides, k_strides, o_strides,
                         scale, kv_len, kv_len_dev, mk, tile_span, tile_ids,
                         o32, m, l, ws, scratch_bytes, stream);
}

extern "C" int dt_flash_fwd_ex(
    const uint16_t* q, const void* k, int k_format, const uint16_t* v,
    const int64_t* v_strides, const uint16_t* vt, int64_t vt_tiles, uint16_t* o,
    int B, int Hq, int Hkv, int Sq, int Skv, int D, const int64_t* q_strides,
    const int64_t* k_strides, const int64_t* o_strides, float scale,
    int kv_len, const int32_t* kv_len_dev, const float* mk,
    const int32_t* tile_span, const int32_t* tile_ids, float* o32, float* m,
    float* l, void* workspace, size_t workspace_bytes, void* stream) {
  if (k_format != 0 && k_format != 1)
    return dt::set_error(DT_ERR_ARG,
                         "dt_flash_fwd_ex: k_format %d (0 bf16, 1 E4M3)",
                         k_format);
  if ((v != nullptr) == (vt != nullptr))
    return dt::set_error(DT_ERR_ARG,
                         "dt_flash_fwd_ex: give exactly one of v and vt");
  return dt::flash_entry(q, k, k_format == 1, v, o, B, Hq, Hkv, Sq, Skv, D,
                         q_strides, k_strides, v_strides, o_strides, scale,
                         kv_len, mk, tile_span, tile_ids, o32, m, l, stream, vt,
                         vt_tiles, workspace, workspace_bytes, kv_len_dev);
}
