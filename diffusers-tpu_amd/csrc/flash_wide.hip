// Flash attention forward for head dim 256 (gfx950): the head dims above
// 128 that kernels/splash.py accepts (it requires only D_v % 8 == 0,
// kernels/splash.py:156-160); dims 136..248 run zero-padded to 256 by the
// Python layer, as the smaller dims pad to 64 or 128.  Same contract as
// flash_attn_kernel (kernels/splash.py:566-650 and the residual form
// :665-742): GQA, a host or device key length (one for the batch or one per
// batch element), residual (o, m, l) outputs, the fixed-m operand.  Not
// here: E4M3 keys, block-sparse tables, packed V and the tail split.
//
// The D = 128 kernel's layout does not fit this width: two wavefronts per
// SIMD leave 256 registers each, and Q^T (64) + O^T (128) + the scores do
// not fit in them.  Here one wavefront runs per SIMD (a workgroup is 4
// wavefronts x 32 query rows), with O^T in the accumulation registers, and
// the key tile is 32 keys, so a ring of 4 stages of K and V stays at
// 128 KiB of LDS.
//   * S^T = K Q^T on v_mfma_f32_32x32x16_bf16, 16 channel steps, Q^T (the
//     query rows scaled by c = scale*log2 e, rounded to bf16) in registers;
//   * lazy exp2-domain softmax as in flash_attn_kernel: a re-base only on
//     the first tile and when a tile's per-lane sum leaves its range, the
//     internal reference 24 below the row's for online heads;
//   * O^T = V^T P^T: the packed probabilities are the B operand; V^T comes
//     from row-major V in LDS through ds_read_b64_tr_b16;
//   * K and V tiles move global -> LDS with buffer_load ... lds, K five and
//     V three tiles ahead of the iteration that first reads them (two rings
//     of 4 stages), the DMA instructions spread over the MFMA slots, one
//     barrier per tile;
//   * a three-stage software pipeline: iteration j interleaves the QK
//     product of tile j+2 with the PV product of tile j, one MFMA of each in
//     turn, and spreads the exponentials of tile j+1 over their slots, one
//     VALU step beside each MFMA.  With one wavefront per SIMD no partner
//     fills the matrix pipe while the softmax runs, so the wavefront's own
//     MFMAs have to.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include <atomic>
#include <type_traits>

#include "../../include/dt_attention.h"
#include "flash_common.h"

namespace dt {
namespace {

constexpr int kWD = 256;                  // head dim
constexpr int kWNW = 4;                   // wavefronts, one per SIMD
constexpr int kWBQ = kWNW * 32;           // 128 query rows per workgroup
constexpr int kWBKV = 32;                 // keys per tile
constexpr int kWStages = 4;               // ring depth, K and V each
constexpr int kWKAhead = 5;               // iteration j requests K of tile j+5
constexpr int kWVAhead = 3;               // ... and V of tile j+3
constexpr int kWRow = 2 * kWD;            // bytes of a K or V row (512)
constexpr int kWTileB = kWBKV * kWRow;    // 16 KiB
constexpr int kWVOff = kWStages * kWTileB;  // V stages after the K stages
constexpr int kWLds = 2 * kWVOff;         // 128 KiB
constexpr int kWLoads = kWTileB / 1024 / kWNW;  // 1 KiB DMAs per wave, K or V
constexpr int kWGroup = 2 * kWLoads;      // DMA instructions per iteration
constexpr int kWSteps = kWD / 16;         // QK channel steps
constexpr int kWNB = kWD / 32;            // 32-channel output blocks
constexpr float kWTrip = 4096.0f;
constexpr float kWShift = 24.0f;          // online heads' reference offset
constexpr float kWTripShifted = kWTrip * 16777216.0f;  // 2^(12 + 24)
constexpr float kWRecenter = 88.0f;       // kernels/fixed_m_bound.py:42
static_assert(kWSteps == 16 && kWNB == 8, "one QK and one PV MFMA per slot");

template <int N>
using WStage = std::integral_constant<int, N>;

__device__ __forceinline__ float dot2_acc(uint32_t w, float acc) {
  const bf16x2 one = {(__bf16)1.0f, (__bf16)1.0f};
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, w), one,
                                         acc, false);
}

// Keeps a value's computation at this point of the instruction stream (the
// empty asm consumes it), so the softmax stays spread over the MFMA slots.
__device__ __forceinline__ void wpin(uint32_t x) { asm volatile("" ::"v"(x)); }
__device__ __forceinline__ void wpin(float x) { asm volatile("" ::"v"(x)); }

// The QK product as inline assembly in the architectural-register form:
// the scores go to the VALU, while the compiler, seeing the O blocks, would
// put every MFMA result of this kernel in the accumulation registers and
// copy the scores out (16 copies per tile, and the register pressure then
// moved Q^T into the accumulation registers as well, 64 more).  The
// compiler does not know these are MFMAs, so it inserts no wait states for
// them: a VALU read of their result must come at least 18 wait states after
// the last one (`mfma_drain`).  Accumulating onto the previous MFMA's result
// in place is supported back to back; the first MFMA of a chain writes
// registers that overlap none of its sources.
__device__ __forceinline__ f32x16 qk_first(bf16x8 a, bf16x8 b,
                                           const f32x16& c) {
  f32x16 d;
  asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %3"
               : "=&v"(d)
               : "v"(a), "v"(b), "v"(c));
  return d;
}
__device__ __forceinline__ void qk_acc(f32x16& d, bf16x8 a, bf16x8 b) {
  asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0"
               : "+v"(d)
               : "v"(a), "v"(b));
}
__device__ __forceinline__ void mfma_drain() {
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
}

// x *= alpha for an O block in the accumulation registers, four elements
// at a time through one temporary.  Written by the compiler, the rare
// re-base copied all 128 O values to the architectural registers at once,
// and the register pressure of that one block moved Q^T into the
// accumulation registers for the whole loop.  Callers drain the MFMA
// pipeline first (mfma_drain); the trailing s_nop covers the accumulation
// register write -> MFMA read wait states of the next accumulation.
__device__ __forceinline__ void scale_acc(f32x16& x, float alpha) {
#pragma unroll
  for (int r = 0; r < 16; r += 4) {
    float a0 = x[r], a1 = x[r + 1], a2 = x[r + 2], a3 = x[r + 3];
    float t;
    asm volatile(
        "v_accvgpr_read_b32 %4, %0\n\tv_mul_f32 %4, %4, %5\n\t"
        "v_accvgpr_write_b32 %0, %4\n\t"
        "v_accvgpr_read_b32 %4, %1\n\tv_mul_f32 %4, %4, %5\n\t"
        "v_accvgpr_write_b32 %1, %4\n\t"
        "v_accvgpr_read_b32 %4, %2\n\tv_mul_f32 %4, %4, %5\n\t"
        "v_accvgpr_write_b32 %2, %4\n\t"
        "v_accvgpr_read_b32 %4, %3\n\tv_mul_f32 %4, %4, %5\n\t"
        "v_accvgpr_write_b32 %3, %4\n\ts_nop 4"
        : "+a"(a0), "+a"(a1), "+a"(a2), "+a"(a3), "=&v"(t)
        : "v"(alpha));
    x[r] = a0;
    x[r + 1] = a1;
    x[r + 2] = a2;
    x[r + 3] = a3;
  }
}

// keys at or past kv_end -> -inf (register r holds key 8(r/4) + 4hf + r%4
// of the tile starting at key kv0)
__device__ __forceinline__ void wide_mask(f32x16& s, int kv0, int hf,
                                          int kv_end) {
  const int lim = kv_end - kv0 - 4 * hf;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int rel = 8 * (r >> 2) + (r & 3);
    if (rel >= lim) s[r] = -INFINITY;
  }
}

__global__ __launch_bounds__(kWNW * 64) void flash_wide_kernel(FlashParams p) {
  extern __shared__ __attribute__((aligned(1024))) uint8_t lds_raw[];
  lds_u8* lds = (lds_u8*)lds_raw;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int l32 = lane & 31;
  const int hf = lane >> 5;

  const int wg = xcd_remap(blockIdx.x, p.n_wg);
  const int qblk = wg % p.n_qblk;
  const int bh = wg / p.n_qblk;
  const int h = bh % p.Hq;
  const int b = bh / p.Hq;
  const int hk = h / (p.Hq / p.Hkv);
  const uint16_t* qbase = p.q + b * p.q_sb + h * p.q_sh;
  const uint16_t* kbase = p.k + b * p.k_sb + hk * p.k_sh;
  const uint16_t* vbase = p.v + b * p.v_sb + hk * p.v_sh;
  const int q0 = qblk * kWBQ + wave * 32;
  const int row = q0 + l32;  // this lane's query row
  const int kv_end =
      resolve_len(p.kv_len_dev, p.kv_len_count, b, p.kv_end, p.Skv);
  const int ntiles = (kv_end + kWBKV - 1) / kWBKV;

  if (ntiles <= 0) {  // no keys (a device length of 0): the empty result
    if (row < p.Sq) {
      const int64_t bhrow = ((int64_t)b * p.Hq + h) * p.Sq + row;
#pragma unroll
      for (int j = 0; j < kWD / 8; ++j) {
        if (p.o32 != nullptr)
          *(u32x4*)(p.o32 + bhrow * kWD + (kWD / 2) * hf + 4 * j) =
              u32x4{0u, 0u, 0u, 0u};
        if (p.o != nullptr)
          *(u32x2*)(p.o + b * p.o_sb + h * p.o_sh + (int64_t)row * p.o_ss +
                    (kWD / 2) * hf + 4 * j) = u32x2{0u, 0u};
      }
      if (p.o32 != nullptr && hf == 0) {
        p.m[bhrow] = 0.f;
        p.l[bhrow] = 0.f;
      }
    }
    return;
  }

  // Q^T: lane holds row `row`, channels 16t + 8hf .. +8 for step t, scaled
  // by c and rounded to bf16 (kernels/splash.py:607-609).  Rows past Sq
  // load row Sq - 1 and are zeroed.
  bf16x8 qf[kWSteps];
  {
    const bool live = row < p.Sq;
    const uint16_t* qrow = qbase + (int64_t)(live ? row : p.Sq - 1) * p.q_ss;
    const uint32_t keep = live ? 0xffffffffu : 0u;
    u32x4 raws[kWSteps];
#pragma unroll
    for (int t = 0; t < kWSteps; ++t)
      raws[t] = *(const u32x4*)(qrow + 16 * t + 8 * hf);
#pragma unroll
    for (int t = 0; t < kWSteps; ++t) {
      u32x4 r = raws[t];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t w = r[e] & keep;
        r[e] = pack_bf16x2(__uint_as_float(w << 16) * p.c,
                           __uint_as_float(w & 0xffff0000u) * p.c);
      }
      qf[t] = __builtin_bit_cast(bf16x8, r);
    }
  }

  // Tile DMA: wave w fills key rows 8w .. 8w+7 of a K or V tile, two
  // 512-byte rows per 1 KiB instruction; lane -> (row 8w + 2i + lane/32,
  // physical 16-byte chunk lane % 32).  K chunk c of key r sits at
  // c ^ (r & 15), V chunk c at c ^ (4 * (r & 3)) (the swizzles of the
  // D = 128 kernel's 256-byte rows, within each 256-byte half).  Tiles at
  // or past the last one are requested too, with an empty range (no memory
  // access; their stages fill with zeros), so every iteration issues the
  // same number of DMA instructions and one vmcnt bound serves all.
  const uint32_t krow = (uint32_t)p.k_ss * 2u;
  const uint32_t vrow = (uint32_t)p.v_ss * 2u;
  uint32_t kvo[kWLoads], vvo[kWLoads];
#pragma unroll
  for (int i = 0; i < kWLoads; ++i) {
    const int r = wave * 8 + 2 * i + (lane >> 5);
    const int pc = lane & 31;
    kvo[i] = r * krow + ((pc ^ (r & 15)) * 16);
    vvo[i] = r * vrow + ((pc ^ (4 * (r & 3))) * 16);
  }
  const uint32_t lds_k = (uint32_t)(uintptr_t)lds + (uint32_t)wave * 8 * kWRow;
  const uint32_t lds_v = lds_k + kWVOff;
  // (wave-uniform; readfirstlane keeps the descriptor in scalar registers,
  // where the compiler would otherwise clamp with a vector instruction)
  auto tile_rows = [&](int t) {
    const int n = kv_end - t * kWBKV;
    return __builtin_amdgcn_readfirstlane(n <= 0 ? 0 : (n < kWBKV ? n : kWBKV));
  };
  // One tile's request: its descriptor (the range ends at kv_end) and LDS
  // stage; `dma` issues the wave's part i of it.
  struct TileReq {
    u32x4 rsrc;
    uint32_t lds;
  };
  auto req_k = [&](int t) {
    const int rows = tile_rows(t);
    const uint64_t base = (uint64_t)(uintptr_t)kbase +
                          (rows > 0 ? (uint64_t)t * kWBKV * krow : 0);
    return TileReq{make_rsrc(base, (uint32_t)rows * krow),
                   lds_k + (uint32_t)(t % kWStages) * kWTileB};
  };
  auto req_v = [&](int t) {
    const int rows = tile_rows(t);
    const uint64_t base = (uint64_t)(uintptr_t)vbase +
                          (rows > 0 ? (uint64_t)t * kWBKV * vrow : 0);
    return TileReq{make_rsrc(base, (uint32_t)rows * vrow),
                   lds_v + (uint32_t)(t % kWStages) * kWTileB};
  };
  auto dma_k = [&](const TileReq& r, int i) {
    lds_dma16_buf(r.rsrc, kvo[i], r.lds + i * 1024);
  };
  auto dma_v = [&](const TileReq& r, int i) {
    lds_dma16_buf(r.rsrc, vvo[i], r.lds + i * 1024);
  };
  auto issue_k = [&](int t) {
    const TileReq r = req_k(t);
#pragma unroll
    for (int i = 0; i < kWLoads; ++i) dma_k(r, i);
  };
  auto issue_v = [&](int t) {
    const TileReq r = req_v(t);
#pragma unroll
    for (int i = 0; i < kWLoads; ++i) dma_v(r, i);
  };

  // Operand offsets within a stage.  K (A operand of S^T): row l32, logical
  // chunk 2t + hf for channel step t; steps t and t + 8 lie 256 bytes
  // apart (the swizzle only touches the chunk's low four bits).  V^T (A
  // operand of O^T) through ds_read_b64_tr_b16: in each 16-lane group g,
  // source lane j names 4 channels of one key (key 4(g >> 1) + j/4,
  // channels 16(g & 1) + 4(j % 4) of the block) and lane i receives channel
  // 16(g & 1) + i of 4 consecutive keys; the read 8 rows further gives the
  // other 4 of the 8 keys the lane's half of the probability operand holds
  // (keys 0-3 and 8-11, or 4-7 and 12-15).  Blocks mb and mb + 4 lie 256
  // bytes apart.  Stage, step and block offsets are compile-time constants
  // (the loop is unrolled over the ring), so they go into the reads'
  // immediate offsets.
  int kread[8];
#pragma unroll
  for (int t = 0; t < 8; ++t)
    kread[t] = l32 * kWRow + (((2 * t + hf) ^ (l32 & 15)) * 16);
  const int g = lane >> 4, j16 = lane & 15;
  const int vkey = 4 * (g >> 1) + (j16 >> 2);
  const int vd0 = 16 * (g & 1) + 4 * (j16 & 3);
  const int vsw = 4 * (vkey & 3);
  int vread[4];
#pragma unroll
  for (int mb = 0; mb < 4; ++mb) {
    const int d0 = 32 * mb + vd0;
    vread[mb] = kWVOff + vkey * kWRow + (((d0 >> 3) ^ vsw) * 16) + (d0 & 7) * 2;
  }
  auto kld = [&](auto stage, int t) {
    constexpr int S = decltype(stage)::value;
    return __builtin_bit_cast(
        bf16x8, *(const __attribute__((address_space(3))) u32x4*)(
                    lds + kread[t & 7] + (S * kWTileB + 256 * (t >> 3))));
  };
  // operand of PV MFMA i: key step i >> 3, output block i & 7
  auto vld = [&](auto stage, int i) {
    constexpr int S = decltype(stage)::value;
    const lds_u8* a = lds + vread[i & 3] +
                      (S * kWTileB + (i >> 3) * 16 * kWRow + 256 * ((i >> 2) & 1));
    const v4i16 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) v4i16*)(a));
    const v4i16 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) v4i16*)(a + 8 * kWRow));
    return __builtin_bit_cast(
        bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
  };

  f32x16 o[kWNB];
#pragma unroll
  for (int mb = 0; mb < kWNB; ++mb)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[mb][r] = 0.f;
  float m = 0.f, l = 0.f;
  bool fixed = false;
  if (p.mk != nullptr && p.mk[p.Hq + h] > 0.5f) {
    fixed = true;
    m = p.mk[h] - kWRecenter;
  }
  const float trip = fixed ? 3.0e38f : kWTripShifted;
  const float shift = fixed ? 0.f : kWShift;
  // QK chains start from -m, so scores come out as c*s - m
  f32x16 negm;
#pragma unroll
  for (int r = 0; r < 16; ++r) negm[r] = -m;

  // Rare path: re-base the lane's row reference on the scores in sc (set
  // it on the first tile of an online head; raise it when the tile's sum
  // leaves its range), recompute their probabilities into pw, shift the
  // already computed next tile's scores sn and rescale l and O.  Then add
  // the tile's sum to l.
  auto settle = [&](bool first, const f32x16& sc, uint32_t (&pw)[8],
                    float sum, f32x16& sn) {
    if (first || wave_any(!(sum <= trip))) {
      mfma_drain();  // sn is written by the QK assembly
      float mx = sc[0];
#pragma unroll
      for (int r = 1; r < 16; ++r) mx = fmaxf(mx, sc[r]);
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      const float delta = first ? mx - shift : fmaxf(mx - shift, 0.f);
      const float alpha = __builtin_amdgcn_exp2f(-delta);
      m += delta;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        negm[r] = -m;
        sn[r] -= delta;
      }
      float sa = 0.f, sb = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        pw[i] = pack_bf16x2(__builtin_amdgcn_exp2f(sc[2 * i] - delta),
                            __builtin_amdgcn_exp2f(sc[2 * i + 1] - delta));
        if (i & 1)
          sb = dot2_acc(pw[i], sb);
        else
          sa = dot2_acc(pw[i], sa);
      }
      sum = sa + sb;
      l *= alpha;
#pragma unroll
      for (int mb = 0; mb < kWNB; ++mb) scale_acc(o[mb], alpha);
    }
    l += sum;
  };

  // ---- prologue: K of tiles 0 and 1, then what iterations -3 and -2
  // would request; S(0) and S(1); after every wave is done with K stage 0,
  // iteration -1's request (K(4) goes there); P(0) with the first re-base.
  issue_k(0);
  issue_k(1);
  issue_k(2);
  issue_v(0);
  issue_k(3);
  issue_v(1);
  wait_vmcnt_c<2 * kWGroup>();  // K(0) and K(1) landed
  __syncthreads();
  f32x16 sA, sB;
  sB = qk_first(kld(WStage<0>{}, 0), qf[0], negm);
  sA = qk_first(kld(WStage<1>{}, 0), qf[0], negm);
#pragma unroll
  for (int t = 1; t < kWSteps; ++t) {
    qk_acc(sB, kld(WStage<0>{}, t), qf[t]);
    qk_acc(sA, kld(WStage<1>{}, t), qf[t]);
  }
  mfma_drain();
  __syncthreads();
  issue_k(4);
  issue_v(2);
  if (kWBKV > kv_end) wide_mask(sB, 0, hf, kv_end);
  if (ntiles > 1 && 2 * kWBKV > kv_end) wide_mask(sA, kWBKV, hf, kv_end);
  uint32_t pwA[8], pwB[8];
  {
    float sa = 0.f, sb = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      pwA[i] = pack_bf16x2(__builtin_amdgcn_exp2f(sB[2 * i]),
                           __builtin_amdgcn_exp2f(sB[2 * i + 1]));
      if (i & 1)
        sb = dot2_acc(pwA[i], sb);
      else
        sa = dot2_acc(pwA[i], sa);
    }
    settle(!fixed, sB, pwA, sa + sb, sA);
  }

  // Iteration j (ring stage S = j % 4 of V, (j + 2) % 4 of K): on entry sc
  // holds S(j+1) and pwc P(j).  32 MFMA slots alternate the QK product of
  // tile j+2 (one accumulator chain into sn) with the PV product of tile j;
  // beside each MFMA one VALU step of P(j+1) (two exps, a pack and a row-sum
  // dot2 per pair of scores) into pwn.  Then the trip check of P(j+1), and
  // the mask of tile j+2 if it is the last, partial one.  When j+2 is past
  // the last tile, QK runs on a zero-filled stage and its scores are never
  // used.
  auto iteration = [&](auto stage, int j, const f32x16& sc, f32x16& sn,
                       const uint32_t (&pwc)[8], uint32_t (&pwn)[8]) {
    constexpr int S = decltype(stage)::value;
    using KS = WStage<(S + 2) % kWStages>;
    wait_vmcnt_c<2 * kWGroup>();  // K(j+2) and V(j) landed (this wave's part)
    mfma_drain();                 // sc was written by the QK assembly
    __syncthreads();              // ... and every wave's; iteration j-1 done
    // K(j+5) goes into the stage K(j+1) used, V(j+3) into the one V(j-1)
    // used; their 8 DMA instructions are spread over the MFMA slots.  Issued
    // together after the barrier, the 32 of the workgroup queued at the
    // CU's address unit for ~500 cycles, and each wavefront, issuing in
    // order, waited behind its own with no MFMA running.
    const TileReq rk = req_k(j + kWKAhead), rv = req_v(j + kWVAhead);
    bf16x8 kr[4], vr[4];
    kr[0] = kld(KS{}, 0);
    vr[0] = vld(stage, 0);
    kr[1] = kld(KS{}, 1);
    vr[1] = vld(stage, 1);
    float sa = 0.f, sb = 0.f, e0 = 0.f, e1 = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      if (i + 2 < 16) {
        kr[(i + 2) & 3] = kld(KS{}, i + 2);
        vr[(i + 2) & 3] = vld(stage, i + 2);
      }
      const int q = i >> 1;
      if (i == 0)
        sn = qk_first(kr[0], qf[0], negm);
      else
        qk_acc(sn, kr[i & 3], qf[i]);
      if (i & 1) {
        pwn[q] = pack_bf16x2(e0, e1);
        wpin(pwn[q]);
        if (i < 8)
          dma_k(rk, i >> 1);
        else
          dma_v(rv, (i - 8) >> 1);
      } else {
        e0 = __builtin_amdgcn_exp2f(sc[2 * q]);
        wpin(e0);
      }
      __builtin_amdgcn_sched_barrier(0);
      const int u = i >> 3, mb = i & 7;
      const u32x4 pr = {pwc[4 * u], pwc[4 * u + 1], pwc[4 * u + 2],
                        pwc[4 * u + 3]};
      o[mb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
          vr[i & 3], __builtin_bit_cast(bf16x8, pr), o[mb], 0, 0, 0);
      if (i & 1) {
        float& acc = (q & 1) ? sb : sa;
        acc = dot2_acc(pwn[q], acc);
        wpin(acc);
      } else {
        e1 = __builtin_amdgcn_exp2f(sc[2 * q + 1]);
        wpin(e1);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    if (j + 1 < ntiles) settle(false, sc, pwn, sa + sb, sn);
    if (j + 2 < ntiles && (j + 3) * kWBKV > kv_end) {
      mfma_drain();
      wide_mask(sn, (j + 2) * kWBKV, hf, kv_end);
    }
  };

  for (int j = 0;; j += 4) {
    iteration(WStage<0>{}, j, sA, sB, pwA, pwB);
    if (j + 1 >= ntiles) break;
    iteration(WStage<1>{}, j + 1, sB, sA, pwB, pwA);
    if (j + 2 >= ntiles) break;
    iteration(WStage<2>{}, j + 2, sA, sB, pwA, pwB);
    if (j + 3 >= ntiles) break;
    iteration(WStage<3>{}, j + 3, sB, sA, pwB, pwA);
    if (j + 4 >= ntiles) break;
  }
  // the requests past the last tile still write their stages: drain them
  // before the workgroup's LDS can go to another workgroup
  wait_vmcnt_c<0>();

  // ---- epilogue: lane holds row `row`, channels 32mb + 8j + 4hf + e of
  // block mb (register 4j + e); the residual (m, l, o) of the reference
  // itself (the online offset taken out)
  if (row >= p.Sq) return;
  const float ltot = l + __shfl_xor(l, 32, 64);
  const float unshift = fixed ? 1.0f : 1.0f / 16777216.0f;  // 2^-kWShift
  const int64_t bhrow = ((int64_t)b * p.Hq + h) * p.Sq + row;
  if (p.o32 != nullptr) {
    float* dst = p.o32 + bhrow * kWD;
#pragma unroll
    for (int mb = 0; mb < kWNB; ++mb)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        f32x4 w;
#pragma unroll
        for (int e = 0; e < 4; ++e) w[e] = o[mb][4 * j + e] * unshift;
        *(f32x4*)(dst + 32 * mb + 8 * j + 4 * hf) = w;
      }
    if (hf == 0) {
      p.m[bhrow] = m + shift;
      p.l[bhrow] = ltot * unshift;
    }
  }
  if (p.o != nullptr) {
    const float inv = 1.0f / ltot;
    uint16_t* dst = p.o + b * p.o_sb + h * p.o_sh + (int64_t)row * p.o_ss;
#pragma unroll
    for (int mb = 0; mb < kWNB; ++mb)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        u32x2 w;
        w[0] = pack_bf16x2(o[mb][4 * j] * inv, o[mb][4 * j + 1] * inv);
        w[1] = pack_bf16x2(o[mb][4 * j + 2] * inv, o[mb][4 * j + 3] * inv);
        *(u32x2*)(dst + 32 * mb + 8 * j + 4 * hf) = w;
      }
  }
}

}  // namespace

int launch_flash_wide(const FlashParams& base, hipStream_t st) {
  if (base.k8 != nullptr || base.vt != nullptr || base.tile_span != nullptr)
    return set_error(DT_ERR_UNSUPPORTED,
                     "dt_flash_fwd: head dim 256 takes bf16 keys, row-major V "
                     "and no tile table");
  FlashParams p = base;
  p.n_qblk = (p.Sq + kWBQ - 1) / kWBQ;
  const int64_t nwg = (int64_t)p.n_qblk * p.Hq * p.B;
  if (nwg > 0x7fffffff)
    return set_error(DT_ERR_SHAPE, "dt_flash_fwd: grid too large");
  // byte offsets of one (b, h) slice's rows are 32-bit in the descriptors
  if ((int64_t)p.kv_end * p.k_ss * 2 >= (1ll << 32) ||
      (int64_t)p.kv_end * p.v_ss * 2 >= (1ll << 32))
    return set_error(DT_ERR_SHAPE, "dt_flash_fwd: K/V slice above 4 GiB");
  p.n_wg = (int)nwg;
  p.n_main = p.n_wg;
  p.n_split = 1;
  p.n_tail = 0;
  p.ws = nullptr;
  static std::atomic<uint64_t> lds_set{0};
  if (int rc = ensure_lds_limit((const void*)flash_wide_kernel, kWLds, lds_set,
                                "dt_flash_fwd"))
    return rc;
  hipLaunchKernelGGL(flash_wide_kernel, dim3(p.n_wg), dim3(kWNW * 64), kWLds,
                     st, p);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return set_error(DT_ERR_LAUNCH, "dt_flash_fwd: %s", hipGetErrorString(e));
  return DT_OK;
}

}  // namespace dt
