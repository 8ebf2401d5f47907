// Flash attention forward for head dims 128 and 64 on gfx950 (bf16 MFMA,
// fp32 softmax).  This is the kernel behind every DiT workload; it replaces
// the reference's splash kernel body (kernels/splash.py:115-375: online
// update :250-267, kv_len masking :216-218 and :277-331, normalize
// :369-375) and its residual form (:665-742).  The notes below give the
// D = 128 figures; at D = 64 rows and tiles are half as wide (128-byte
// rows, 64 KiB of LDS) and each MFMA of a phase carries more of the
// softmax.
//
// Decomposition
//   * One workgroup = 8 wavefronts = 256 query rows of one (batch, head);
//     wavefront w owns rows 32w .. 32w+31 for the whole key sweep.  Waves w
//     and w+4 share a SIMD.
//   * Keys/values stream through LDS in 64-key tiles, a ring of 4 (K, V)
//     stages (128 KiB: the four K tiles, then the four V tiles).  Tile t is
//     requested two iterations before its QK step with
//     buffer_load_dwordx4 ... lds (global -> LDS, no VGPR staging) through
//     per-tile buffer descriptors: all per-tile address work is scalar, and
//     the descriptor's range ends at kv_len so rows past it arrive as
//     zeros.  One barrier per tile.  The key loop is unrolled over the
//     ring, so each LDS operand address is a per-lane register plus a
//     constant immediate.
//   * LDS rows are unpadded (256 B) with 16-byte chunks XOR-swizzled per
//     row, so that every operand read is bank-conflict free:
//       K chunk c of key r lives at chunk c ^ (r & 15)
//       V chunk c of key r lives at chunk c ^ (4 * (r & 3))
//     V may instead come packed (VT; dt_pack_v): per tile a 128-channel x
//     64-key block, chunk c of channel row d at c ^ ((d >> 1) & 7), keys
//     in the score accumulator's order, so a V^T operand is one
//     ds_read_b128.
//   * A query block of a partly filled last round of workgroups may run as
//     a split part (n_split > 1): a contiguous share of its key tiles, with
//     unnormalized o, m, l written to the workspace for split_merge_kernel.
//   * Scores are computed transposed, S^T = K Q^T (v_mfma_f32_32x32x16_bf16;
//     A = K from LDS, one ds_read_b128 per 32x16 block; B = Q^T held in
//     registers).  In the 32x32 accumulator lane l holds one query row
//     (column l%32) and 32 of the tile's 64 keys; the other 32 keys of that
//     row sit in lane l^32.  The output is accumulated transposed too,
//     O^T = V^T P^T: the probabilities, packed to bf16, are directly the B
//     operand, so they never leave registers.  With row-major V the V^T
//     operand comes from ds_read_b64_tr_b16, which transposes in flight: in each
//     16-lane group, source lane j names 4 channels of one key (key =
//     kbase + j/4, channels dbase + 4*(j%4) .. +3) and lane i receives
//     channel dbase + i of keys kbase .. kbase+3.  Two such reads give the
//     8 keys a lane half holds in the score accumulator.
//   * Per key tile j a wavefront runs
//       phase A: S(j+1) = K(j+1) Q^T, its 16 MFMAs interleaved with the
//                exp2 / bf16 packing / row sum of pairs 8..15 of the 16
//                score pairs of tile j that this lane holds;
//       phase B: O += V(j)^T P(j)^T (16 MFMAs), interleaved with pairs
//                0..7 of tile j+1,
//     with operand reads two steps ahead and scheduling fences keeping the
//     order.  The VALU work runs in the shadow of the MFMAs.
//   * Softmax in the exp2 domain with lazy rescaling.  q is pre-scaled by
//     c = scale*log2 e (and rounded to bf16, as the reference folds the
//     scale into q) and each QK accumulator starts at -m, the row's current
//     reference, so the MFMAs emit c*s - m and p = exp2(score) is one
//     instruction.  m moves, with the O/l rescale, on the first tile and
//     when a tile's per-lane sum of p exceeds 2^12 or is not finite (a large
//     new maximum).  The result is the exact softmax; the common path has no
//     row max and no O rescale.  Row sums use v_dot2_f32_bf16 on the packed
//     probabilities, i.e. the same bf16 weights the PV product uses.
//   * The epilogue stages each wave's output rows through a ring stage the
//     last iteration does not read and stores whole rows (16 contiguous
//     bytes per lane) instead of the accumulator layout's 16-byte pieces
//     of 32 rows per instruction.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include <atomic>
#include <type_traits>

#include "../../include/dt_attention.h"
#include "flash_common.h"

namespace dt {
namespace {

constexpr int kNW = 8;               // wavefronts per workgroup
constexpr int kBQ = kNW * 32;        // query rows per workgroup
constexpr int kBKV = 64;             // keys per tile
constexpr int kNStage = 4;           // LDS ring depth
// Tiles requested ahead of their use.  Two: three kept a third tile per CU
// in flight and measured 0.2-0.7 % slower with bf16 keys (V7, V4, I1, I2,
// two boxes) and 3.3 % slower with E4M3 keys at V7, the deeper DMA queue
// lengthening every tile's latency; with two, one stage of the ring is
// always idle.
constexpr int kDist = 2;
constexpr int kRowsPerWave = kBKV / kNW;  // tile rows each wave loads

// LDS layout for head dim D: the K tiles of the 4 ring stages (bf16: 2D-byte
// rows; E4M3: D-byte rows), then the 4 V tiles (2D-byte key rows, or with
// packed V 128 channel rows of 128 B).  Every operand address is then a
// per-lane register plus a compile-time offset below 64 KiB (the key loop
// is unrolled over the ring, so the stage is a constant), which the LDS
// read encodes as its immediate offset: no per-tile address arithmetic.
// QK8 selects E4M3 keys (the reference's qk_fp8).
template <int D, bool QK8>
struct Stage {
  static constexpr int kKRow = QK8 ? D : 2 * D;  // bytes of a K row
  static constexpr int kVRow = 2 * D;            // bytes of a V key row
  static constexpr int kKTileB = kBKV * kKRow;
  static constexpr int kVTileB = kBKV * kVRow;
  static constexpr int kVOff = kNStage * kKTileB;
  static constexpr int kLds = kVOff + kNStage * kVTileB;
  // 1 KiB DMA instructions per wave per tile
  static constexpr int kKLoads = kKTileB / 1024 / kNW;
  static constexpr int kVLoads = kVTileB / 1024 / kNW;
  static constexpr int kLoadsPerTile = kKLoads + kVLoads;
  static constexpr int kSteps = D / 16;  // k-steps of a bf16 QK product
  static constexpr int kNB = D / 32;     // 32-channel output blocks
};
constexpr float kTripSum = 4096.0f;
// Online heads keep their internal reference kPShift below the row
// reference m (scores come out as c*s - m + kPShift, probabilities are
// 2^kPShift times the reference ones, up to 2^(12 + kPShift) before a
// re-base); the epilogue takes the factor back out of l, o and m.  The
// results are the same up to rounding of the scores; at V7 the kernel
// measured 1.1 % faster with it at the power limit (16 to 63 alike, 8
// half of that): probabilities around 2^0 are a costlier MFMA operand than
// the same values scaled by a power of two.  Fixed-m heads already run at
// up to 2^88 and keep their reference unshifted.
constexpr float kPShift = 24.0f;
constexpr float kTripShifted = kTripSum * 16777216.0f;  // 2^(12 + 24)
constexpr int kMaxSplit = 16;       // most parts a query block is split into
template <int N>
using IC = std::integral_constant<int, N>;  // a compile-time ring stage
constexpr float kFixedRecenter = 88.0f;  // kernels/fixed_m_bound.py:42

// scores of keys at or past kv_end -> -inf.  Bit arithmetic (a sign mask
// and a bitfield select) rather than 32 compares, which would each claim a
// scalar register pair.
__device__ __forceinline__ void mask_tile(f32x16 (&s)[2], int kv0, int hf,
                                          int kv_end) {
  const int lim = kv_end - kv0 - 4 * hf;  // key offsets below lim are valid
#pragma unroll
  for (int kb = 0; kb < 2; ++kb)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int rel = kb * 32 + 8 * (r >> 2) + (r & 3);
      const uint32_t keep = (uint32_t)((rel - lim) >> 31);  // all ones: valid
      const uint32_t bits = __float_as_uint(s[kb][r]);
      s[kb][r] = __uint_as_float((bits & keep) | (0xff800000u & ~keep));
    }
}

// probabilities of pair i (scores 2i, 2i+1 of the lane's 32), packed.  The
// scores already hold c*s - m (see the QK accumulator), so p = exp2(score).
__device__ __forceinline__ uint32_t exp_pair(const f32x16 (&s)[2], int i) {
  return pack_bf16x2(__builtin_amdgcn_exp2f(s[i >> 3][(2 * i) & 15]),
                     __builtin_amdgcn_exp2f(s[i >> 3][(2 * i + 1) & 15]));
}

// Pins the computation of x at this point of the instruction stream: the
// empty asm consumes it, so the compiler can neither sink the producing
// instructions into a later block (it moved the probabilities of one phase
// past the loop's branches into the next phase) nor drop the interleave.
__device__ __forceinline__ void pin(uint32_t x) { asm volatile("" ::"v"(x)); }
__device__ __forceinline__ void pin(float x) { asm volatile("" ::"v"(x)); }

__device__ __forceinline__ float dot2_sum(uint32_t w, float acc) {
  const bf16x2 one = {(__bf16)1.0f, (__bf16)1.0f};
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, w), one,
                                         acc, false);
}

// Rare path: raise the reference m of the lane's row to the row max of the
// tile in s (on the first tile: set it to that max), re-base the scores of s
// and of the already computed next tile sn, recompute the probabilities of s
// and rescale l and O.  Scores are relative to the old m on entry.
template <int NB>
__device__ __forceinline__ float softmax_fixup(f32x16 (&s)[2], f32x16 (&sn)[2],
                                               bool first, float& m, float& l,
                                               f32x16& negm, uint32_t (&pw)[16],
                                               f32x16 (&o)[NB], float shift) {
  float mx = s[0][0];
#pragma unroll
  for (int kb = 0; kb < 2; ++kb)
#pragma unroll
    for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[kb][r]);
  mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
  // (scores are relative to m - shift: the row's max is mx - shift above m)
  const float delta = first ? mx - shift : fmaxf(mx - shift, 0.f);
  const float alpha = __builtin_amdgcn_exp2f(-delta);
  m += delta;
#pragma unroll
  for (int r = 0; r < 16; ++r) negm[r] = -m;
#pragma unroll
  for (int kb = 0; kb < 2; ++kb)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      s[kb][r] -= delta;
      sn[kb][r] -= delta;
    }
  float sa = 0.f, sb = 0.f;
#pragma unroll
  for (int i = 0; i < 16; i += 2) {
    pw[i] = exp_pair(s, i);
    pw[i + 1] = exp_pair(s, i + 1);
    sa = dot2_sum(pw[i], sa);
    sb = dot2_sum(pw[i + 1], sb);
  }
  l *= alpha;
#pragma unroll
  for (int mb = 0; mb < NB; ++mb)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[mb][r] *= alpha;
  return sa + sb;
}

}  // namespace

template <int D, bool QK8, bool SPARSE, bool VT>
__global__ __launch_bounds__(kNW * 64) void flash_attn_kernel(FlashParams p) {
  // head dim 64 runs the dense bf16 row-major-V form only
  static_assert(D == 128 || (D == 64 && !QK8 && !SPARSE && !VT),
                "unsupported head dim / variant");
  using L = Stage<D, QK8>;
  constexpr int NB = L::kNB;
  extern __shared__ __attribute__((aligned(1024))) uint8_t lds_raw[];
  lds_u8* lds = (lds_u8*)lds_raw;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int l32 = lane & 31;
  const int hf = lane >> 5;

  // tail split: unit >= 0 names (query block, part) of a split workgroup
  int wg, unit = -1, part = 0;
  if ((int)blockIdx.x < p.n_main) {
    wg = xcd_remap(blockIdx.x, p.n_main);
  } else {
    unit = blockIdx.x - p.n_main;
    wg = p.n_main + unit / p.n_split;
    part = unit - (unit / p.n_split) * p.n_split;
  }
  const int qblk = wg % p.n_qblk;
  const int bh = wg / p.n_qblk;
  const int h = bh % p.Hq;
  const int b = bh / p.Hq;
  const int hk = h / (p.Hq / p.Hkv);

  const uint16_t* qbase = p.q + b * p.q_sb + h * p.q_sh;
  // K row bytes: E4M3 keys are one byte per element
  const uint8_t* kbase =
      QK8 ? p.k8 + b * p.k_sb + hk * p.k_sh
          : (const uint8_t*)(p.k + b * p.k_sb + hk * p.k_sh);
  const uint16_t* vbase =
      VT ? p.vt + ((int64_t)b * p.Hkv + hk) * p.vt_tiles * (kBKV * D)
         : p.v + b * p.v_sb + hk * p.v_sh;
  const int q0 = qblk * kBQ + wave * 32;
  const float c = p.c;
  const int kv_end =
      resolve_len(p.kv_len_dev, p.kv_len_count, b, p.kv_end, p.Skv);
  // Key tiles this (head, query block) visits: all of [0, kv_end), or with
  // a block-sparse table the listed 64-key tiles (sparse_splash.py:426-427).
  // The table is read through the constant address space, i.e. with scalar
  // loads: a vector load would count in vmcnt, which tracks the tile DMA.
  typedef const __attribute__((address_space(4))) int32_t cint32;
  int ntiles = (kv_end + kBKV - 1) / kBKV;
  cint32* tiles = nullptr;
  if constexpr (SPARSE) {
    cint32* sp = (cint32*)p.tile_span + 2 * ((int64_t)h * p.n_qblk + qblk);
    tiles = (cint32*)p.tile_ids + sp[0];
    ntiles = __builtin_amdgcn_readfirstlane(sp[1] - sp[0]);
  }
  // a split part visits a contiguous share of the block's tiles
  int tbeg = 0;
  if (unit >= 0) {
    tbeg = (ntiles * part) / p.n_split;
    ntiles = (ntiles * (part + 1)) / p.n_split - tbeg;
  }
  auto tile_of = [&](int j) {
    if constexpr (SPARSE)
      return __builtin_amdgcn_readfirstlane(tiles[tbeg + j]);
    return tbeg + j;
  };
  // outputs: a split part writes o (unnormalized), m and l of its rows to
  // the workspace, row unit*256 + (row - qblk*256)
  float* out32 = p.o32;
  float* out_m = p.m;
  float* out_l = p.l;
  uint16_t* out_o = p.o;
  if (unit >= 0) {
    const int64_t units = (int64_t)p.n_tail * p.n_split;
    out32 = p.ws;
    out_m = p.ws + units * kBQ * D;
    out_l = out_m + units * kBQ;
    out_o = nullptr;
  }
  auto out_row = [&](int row) -> int64_t {  // index of row in out32/m/l
    if (unit >= 0) return (int64_t)unit * kBQ + (row - qblk * kBQ);
    return ((int64_t)b * p.Hq + h) * p.Sq + row;
  };
  // an empty table row, or a split part past a runtime kv_len: nothing to
  // attend to
  if (ntiles <= 0) {
    const int row = q0 + l32;
    if (row < p.Sq) {
      const int64_t bhrow = out_row(row);
      // this lane's half of the row: D/2 channels from D/2 * hf
#pragma unroll
      for (int j = 0; j < D / 8; ++j) {
        if (out32 != nullptr)
          *(u32x4*)(out32 + bhrow * D + (D / 2) * hf + 4 * j) = u32x4{0u, 0u, 0u, 0u};
        if (out_o != nullptr)
          *(u32x2*)(out_o + b * p.o_sb + h * p.o_sh + (int64_t)row * p.o_ss +
                    (D / 2) * hf + 4 * j) = u32x2{0u, 0u};
      }
      if (out32 != nullptr && hf == 0) {
        out_m[bhrow] = 0.f;
        out_l[bhrow] = 0.f;
      }
    }
    return;
  }

  // ---- Q^T operands, in registers for the whole sweep: lane holds row
  // q0 + l32, channels 16t + 8hf .. +8 for step t.  They are pre-scaled by
  // c = scale*log2(e) and rounded back to bf16, as the reference folds the
  // scale into q before the kernel (kernels/splash.py:607-609).
  // With QK8 the scaled bf16 values are then cast to E4M3, saturating at
  // +-448 (kernels/fp8_cast.py:28-39): lane holds channels 64t + 32hf .. +32
  // of its row for step t, one byte each, in channel order.
  bf16x8 qf[L::kSteps];
  i32x8 qf8[2];
  {
    // Rows past Sq load row Sq-1 (in bounds) and are zeroed after: loads
    // under a per-row branch were issued in two dependent batches (the
    // compiler waited for the first two before issuing the rest), one
    // more memory round trip in every workgroup's start-up.
    const int row = q0 + l32;
    const bool live = row < p.Sq;
    const uint16_t* qrow = qbase + (int64_t)(live ? row : p.Sq - 1) * p.q_ss;
    auto qload = [&](int off) {
      const u32x4 r = *(const u32x4*)(qrow + off);
      const uint32_t keep = live ? 0xffffffffu : 0u;
      return u32x4{r[0] & keep, r[1] & keep, r[2] & keep, r[3] & keep};
    };
    if constexpr (!QK8) {
      u32x4 raws[L::kSteps];
#pragma unroll
      for (int t = 0; t < L::kSteps; ++t) raws[t] = qload(16 * t + 8 * hf);
#pragma unroll
      for (int t = 0; t < L::kSteps; ++t) {
        u32x4 raw = raws[t];
#pragma unroll
        for (int e = 0; e < 4; ++e)
          raw[e] = pack_bf16x2(__uint_as_float(raw[e] << 16) * c,
                               __uint_as_float(raw[e] & 0xffff0000u) * c);
        qf[t] = __builtin_bit_cast(bf16x8, raw);
      }
    } else {
      u32x4 raws[8];
#pragma unroll
      for (int i = 0; i < 8; ++i)
        raws[i] = qload(64 * (i >> 2) + 32 * hf + 8 * (i & 3));
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const u32x4 raw = raws[4 * t + u];
#pragma unroll
          for (int e = 0; e < 2; ++e) {
            // channels 8u + 4e .. +3 -> dword 2u + e
            const uint32_t w0 = pack_bf16x2(__uint_as_float(raw[2 * e] << 16) * c,
                                            __uint_as_float(raw[2 * e] & 0xffff0000u) * c);
            const uint32_t w1 = pack_bf16x2(__uint_as_float(raw[2 * e + 1] << 16) * c,
                                            __uint_as_float(raw[2 * e + 1] & 0xffff0000u) * c);
            qf8[t][2 * u + e] = pack_e4m3x4(w0, w1);
          }
        }
    }
  }

  // ---- tile loads: wave w fills rows 8w .. 8w+7 of the K and V tiles;
  // lane -> (row, physical chunk).  256-byte rows (bf16 K and V at
  // D = 128): 4 rows per 1 KiB instruction, K chunk c of key r at
  // c ^ (r & 15), V chunk c at c ^ (4 * (r & 3)).  128-byte rows (E4M3 K,
  // and bf16 K and V at D = 64): 8 rows per instruction; two rows share
  // each 256-byte bank cycle, so the swizzles follow row pairs: K chunk c
  // at c ^ ((r >> 1) & 7), which keeps every 16 consecutive rows of one
  // logical chunk on distinct banks, V chunk c at c ^ (4 * ((r >> 1) & 1)),
  // which keeps the transposing reads' four rows per half-wave apart.
  const uint32_t krow = (uint32_t)p.k_ss * (QK8 ? 1u : 2u);
  // V row bytes: a key row, or with packed V a channel row of one tile
  const uint32_t vrow = VT ? (uint32_t)kBKV * 2u : (uint32_t)p.v_ss * 2u;
  uint32_t kvo[L::kKLoads], vvo[L::kVLoads];
  {
    if constexpr (L::kKRow == 256) {
#pragma unroll
      for (int i = 0; i < L::kKLoads; ++i) {
        const int row = wave * kRowsPerWave + i * 4 + (lane >> 4);
        kvo[i] = row * krow + (((lane & 15) ^ (row & 15)) * 16);
      }
    } else {
      const int row = wave * kRowsPerWave + (lane >> 3);
      kvo[0] = row * krow + (((lane & 7) ^ ((row >> 1) & 7)) * 16);
    }
    if constexpr (VT) {
      // packed V tile: 128 channel rows x 128 B (64 keys); wave w fills
      // rows 16w .. 16w+15, 8 rows per instruction; chunk c of row d at
      // c ^ ((d >> 1) & 7), as the E4M3 K tile
#pragma unroll
      for (int i = 0; i < L::kVLoads; ++i) {
        const int row = wave * 16 + i * 8 + (lane >> 3);
        vvo[i] = row * vrow + (((lane & 7) ^ ((row >> 1) & 7)) * 16);
      }
    } else if constexpr (L::kVRow == 256) {
#pragma unroll
      for (int i = 0; i < L::kVLoads; ++i) {
        const int row = wave * kRowsPerWave + i * 4 + (lane >> 4);
        vvo[i] = row * vrow + (((lane & 15) ^ (4 * (row & 3))) * 16);
      }
    } else {
      const int row = wave * kRowsPerWave + (lane >> 3);
      vvo[0] = row * vrow + (((lane & 7) ^ (4 * ((row >> 1) & 1))) * 16);
    }
  }
  const uint32_t lds_k = (uint32_t)(uintptr_t)lds +
                         (uint32_t)wave * (kRowsPerWave * L::kKRow);
  // (a packed V tile's wave share, 16 rows of 128 B, is 8 rows of 256 B)
  const uint32_t lds_v = (uint32_t)(uintptr_t)lds + L::kVOff +
                         (uint32_t)wave * (kRowsPerWave * L::kVRow);
  // t: position in the visit order (selects the LDS stage); kt: key tile
  // The request of the tile at visit position t (key tile kt): descriptors
  // and LDS stages.  An invalid request (past the last tile) has empty
  // ranges: its DMAs read nothing and fill their stage with zeros.
  struct TileReq {
    u32x4 rk, rv;
    uint32_t sk, sv;
  };
  auto tile_req = [&](bool valid, int t, int kt) {
    const int kv0 = kt * kBKV;
    int rows = kv_end - kv0 < kBKV ? kv_end - kv0 : kBKV;
    // a listed tile may start past kv_end; readfirstlane keeps the clamp,
    // which the compiler forms as a vector med3, out of the scalar descriptor
    if constexpr (SPARSE) rows = __builtin_amdgcn_readfirstlane(rows < 0 ? 0 : rows);
    if (!valid) rows = 0;
    TileReq r;
    r.rk = make_rsrc((uint64_t)(uintptr_t)kbase + (uint64_t)kv0 * krow,
                     (uint32_t)rows * krow);
    // a packed V tile is one contiguous 16 KiB block, zero past kv_end
    r.rv = VT ? make_rsrc((uint64_t)(uintptr_t)vbase + (uint64_t)kt * L::kVTileB,
                          valid ? (uint32_t)L::kVTileB : 0u)
              : make_rsrc((uint64_t)(uintptr_t)vbase + (uint64_t)kv0 * vrow,
                          (uint32_t)rows * vrow);
    r.sk = lds_k + (uint32_t)(t % kNStage) * L::kKTileB;
    r.sv = lds_v + (uint32_t)(t % kNStage) * L::kVTileB;
    return r;
  };
  // DMA instruction `part` of a request: the K parts first (K is read one
  // phase earlier than V: 0.25-0.45 % at V7 against interleaving the two)
  auto dma_part = [&](const TileReq& r, int part) {
    if (part < L::kKLoads)
      lds_dma16_buf(r.rk, kvo[part], r.sk + part * 1024);
    else
      lds_dma16_buf(r.rv, vvo[part - L::kKLoads],
                    r.sv + (part - L::kKLoads) * 1024);
  };
  auto issue_tile = [&](int t, int kt) {
    const TileReq r = tile_req(true, t, kt);
#pragma unroll
    for (int i = 0; i < L::kLoadsPerTile; ++i) dma_part(r, i);
  };
  // wait until at most `pending` tiles of this wave's loads are in flight,
  // then make every wave's loads visible
  auto wait_tiles = [&](int pending) {
    wait_vmcnt(pending * L::kLoadsPerTile);
    __syncthreads();
  };

  // ---- per-lane LDS operand offsets (bytes within a stage)
  // K: step t, key block kb: row kb*32 + l32, chunk 2t + hf (kb adds 8 KiB)
  // E4M3 K: step t (64 channels), half e: row kb*32 + l32, chunk
  // 4t + 2hf + e (kb adds 4 KiB)
  // K at D = 64: step t, key block kb: row kb*32 + l32, chunk 2t + hf at
  // (2t + hf) ^ ((l32 >> 1) & 7) (kb adds 4 KiB)
  int kread[L::kSteps];
#pragma unroll
  for (int t = 0; t < L::kSteps; ++t)
    kread[t] = QK8 ? l32 * 128 +
                         ((((t >> 1) * 4 + 2 * hf + (t & 1)) ^ ((l32 >> 1) & 7)) * 16)
             : L::kKRow == 256 ? l32 * 256 + (((2 * t + hf) ^ (l32 & 15)) * 16)
                               : l32 * 128 + (((2 * t + hf) ^ ((l32 >> 1) & 7)) * 16);
  // V^T: channel block mb, key step u (adds 4 KiB), read half e (adds 2 KiB)
  // Packed V: key step u, channel block mb (adds 4 KiB): row 32mb + l32,
  // logical chunk 2u + hf, at physical chunk (2u + hf) ^ ((l32 >> 1) & 7)
  int vread[4];
  if constexpr (VT) {
    const int sw = (l32 >> 1) & 7;
#pragma unroll
    for (int u = 0; u < 4; ++u)
      vread[u] = L::kVOff + l32 * 128 + (((2 * u + hf) ^ sw) * 16);
  } else {
    const int g = lane >> 4, j16 = lane & 15;
    const int vkey = 4 * (g >> 1) + (j16 >> 2);
    const int vd0 = 16 * (g & 1) + 4 * (j16 & 3);
    // (a 16-key step adds 16 rows and the read half 8: neither changes
    // the swizzle of 128-byte rows, which follows (row >> 1) & 1)
    const int vsw = L::kVRow == 256 ? 4 * (vkey & 3) : 4 * ((vkey >> 1) & 1);
#pragma unroll
    for (int mb = 0; mb < NB; ++mb) {
      const int d0 = 32 * mb + vd0;
      vread[mb] = L::kVOff + vkey * L::kVRow + (((d0 >> 3) ^ vsw) * 16) +
                  (d0 & 7) * 2;
    }
  }

  f32x16 o[NB];
#pragma unroll
  for (int mb = 0; mb < NB; ++mb)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[mb][r] = 0.f;
  // m: the lane's row reference (log2 units); the QK accumulators start at
  // -m, so scores come out as c*s - m.  Online heads re-base m on the first
  // tile; a fixed-m head starts from its bound minus the recentering
  // constant (probabilities up to 2^88, kernels/splash.py:170-196) and
  // re-bases only when a sum overflows.
  float m = 0.f, l = 0.f;
  bool fixed = false;
  if (p.mk != nullptr && p.mk[p.Hq + h] > 0.5f) {
    fixed = true;
    m = p.mk[h] - kFixedRecenter;
  }
  const float trip = fixed ? 3.0e38f : kTripShifted;
  const float shift = fixed ? 0.f : kPShift;
  f32x16 negm;
#pragma unroll
  for (int r = 0; r < 16; ++r) negm[r] = -m;
  uint32_t pw[16];

  // Phase A: S of the tile in ring stage STAGE into sn; with SOFTMAX,
  // interleave the probabilities of the scores in sc (into pw) and return
  // their per-lane sum.
  // `dma(i)` issues the tile DMA instructions scheduled beside MFMA i.
  auto phase_a = [&](auto softmax, auto stage, f32x16 (&sn)[2],
                     const f32x16 (&sc)[2], auto&& dma) -> float {
    constexpr bool SM = decltype(softmax)::value;
    const lds_u8* kt = lds + decltype(stage)::value * L::kKTileB;
    const lds_u8* kp[L::kSteps];
#pragma unroll
    for (int st = 0; st < L::kSteps; ++st) kp[st] = kt + kread[st];
    auto kld = [&](int i) {
      return __builtin_bit_cast(
          bf16x8, *(const __attribute__((address_space(3))) u32x4*)(
                      kp[i >> 1] + (i & 1) * 32 * L::kKRow));
    };
    float sa = 0.f, sb = 0.f;
    if constexpr (QK8) {
      // 4 MFMAs 32x32x64 on E4M3: step i >> 1 (64 channels), key block
      // i & 1; two pairs of probabilities of sc in the shadow of each
      auto kld8 = [&](int i) {
        const lds_u8* a = kt + kread[2 * (i >> 1)] + (i & 1) * 32 * 128;
        const lds_u8* a2 = kt + kread[2 * (i >> 1) + 1] + (i & 1) * 32 * 128;
        const u32x4 lo = *(const __attribute__((address_space(3))) u32x4*)a;
        const u32x4 hi = *(const __attribute__((address_space(3))) u32x4*)a2;
        return __builtin_bit_cast(
            i32x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
      };
      i32x8 kr8[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) kr8[i] = kld8(i);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        sn[i & 1] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
            kr8[i], qf8[i >> 1], i < 2 ? negm : sn[i & 1], 0, 0, 0, 0, 0, 0);
        if constexpr (SM) {
          pw[8 + 2 * i] = exp_pair(sc, 8 + 2 * i);
          sa = dot2_sum(pw[8 + 2 * i], sa);
          pw[9 + 2 * i] = exp_pair(sc, 9 + 2 * i);
          sb = dot2_sum(pw[9 + 2 * i], sb);
          pin(pw[8 + 2 * i]);
          pin(pw[9 + 2 * i]);
          pin(sa);
          pin(sb);
        }
        dma(i);
        __builtin_amdgcn_sched_barrier(0);
      }
      return sa + sb;
    }
    // 2*kSteps MFMAs (16 at D = 128, 8 at D = 64), the 8 probability pairs
    // of sc spread evenly over them
    constexpr int NM = 2 * L::kSteps, EVERY = NM / 8;
    bf16x8 kr[4];
    kr[0] = kld(0);
    kr[1] = kld(1);
#pragma unroll
    for (int i = 0; i < NM; ++i) {
      if (i + 2 < NM) kr[(i + 2) & 3] = kld(i + 2);
      if (i < 2) {
        sn[i & 1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kr[i & 3], qf[i >> 1],
                                                            negm, 0, 0, 0);
      } else {
        sn[i & 1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
            kr[i & 3], qf[i >> 1], sn[i & 1], 0, 0, 0);
      }
      if constexpr (SM) {
        if (i % EVERY == EVERY - 1) {
          // two running sums halve the dependent dot2 chain
          const int pi = 8 + i / EVERY;
          pw[pi] = exp_pair(sc, pi);
          float& acc = ((i / EVERY) & 1) ? sb : sa;
          acc = dot2_sum(pw[pi], acc);
          pin(pw[pi]);
          pin(acc);
        }
      }
      dma(i);
      __builtin_amdgcn_sched_barrier(0);
    }
    return sa + sb;
  };
  auto no_dma = [](int) {};
  // probabilities of pairs first .. first+7 of sc with no MFMAs to hide
  // them under (the first half of tile 0, before the loop)
  auto softmax_half = [&](const f32x16 (&sc)[2], int first) -> float {
    float sa = 0.f, sb = 0.f;
#pragma unroll
    for (int i = 0; i < 8; i += 2) {
      pw[first + i] = exp_pair(sc, first + i);
      pw[first + i + 1] = exp_pair(sc, first + i + 1);
      sa = dot2_sum(pw[first + i], sa);
      sb = dot2_sum(pw[first + i + 1], sb);
    }
    return sa + sb;
  };
  // Phase B: O += V^T P^T for the tile in ring stage STAGE, V^T operands
  // two steps ahead
  auto phase_b = [&](auto softmax, auto stage, const f32x16 (&sn)[2],
                     float& hs, auto&& dma) {
    constexpr bool SMB = decltype(softmax)::value;
    float h0 = 0.f, h1 = 0.f;
    // (the V base is in vread: the stage offset alone fits the immediate)
    const lds_u8* st = lds + decltype(stage)::value * L::kVTileB;
    const lds_u8* vp[4];
#pragma unroll
    for (int mb = 0; mb < (VT ? 4 : NB); ++mb) vp[mb] = st + vread[mb];
    // MFMA i: key step u = i / NB, output block mb = i % NB
    auto vld = [&](int i) {
      if constexpr (VT)  // one 16-byte read: step i >> 2, block i & 3
        return __builtin_bit_cast(
            bf16x8, *(const __attribute__((address_space(3))) u32x4*)(
                        vp[i >> 2] + (i & 3) * 32 * 128));
      const lds_u8* a = vp[i % NB] + (i / NB) * 16 * L::kVRow;
      const v4i16 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (__attribute__((address_space(3))) v4i16*)(a));
      const v4i16 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (__attribute__((address_space(3))) v4i16*)(a + 8 * L::kVRow));
      return __builtin_bit_cast(
          bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
    };
    // pairs 0..7 of sn go into pw once the MFMAs that read the current
    // tile's pw words have issued: pw[4u..4u+3] is read by key step u, so
    // pairs 0..3 may follow step 0 and pairs 4..7 step 1.  D = 128: one
    // pair on each of MFMAs 4..11; D = 64: two on each of MFMAs 2..5.
    constexpr int NMB = 4 * NB, PPM = NB == 4 ? 1 : 2, P0 = NB;
    bf16x8 vr[4];
    vr[0] = vld(0);
    vr[1] = vld(1);
#pragma unroll
    for (int i = 0; i < NMB; ++i) {
      if (i + 2 < NMB) vr[(i + 2) & 3] = vld(i + 2);
      const int u = i / NB, mb = i % NB;
      const u32x4 pr = {pw[4 * u], pw[4 * u + 1], pw[4 * u + 2], pw[4 * u + 3]};
      o[mb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
          vr[i & 3], __builtin_bit_cast(bf16x8, pr), o[mb], 0, 0, 0);
      if constexpr (SMB) {
        if (i >= P0 && i < P0 + 8 / PPM) {
#pragma unroll
          for (int e = 0; e < PPM; ++e) {
            const int pi = (i - P0) * PPM + e;
            pw[pi] = exp_pair(sn, pi);
            float& acc = (pi & 1) ? h1 : h0;
            acc = dot2_sum(pw[pi], acc);
            pin(pw[pi]);
            pin(acc);
          }
        }
      }
      dma(i);
      __builtin_amdgcn_sched_barrier(0);
    }
    hs = h0 + h1;
  };

  using T = std::true_type;
  using F = std::false_type;



  // ---- prologue: tiles 0 .. kDist-1 requested, S(0)
#pragma unroll
  for (int t = 0; t < kDist; ++t)
    if (t < ntiles) issue_tile(t, tile_of(t));
  wait_tiles(ntiles - 1 < kDist - 1 ? ntiles - 1 : kDist - 1);
  f32x16 sA[2], sB[2];
  phase_a(F{}, IC<0>{}, sA, sA, no_dma);
  {
    const int k0 = tile_of(0) * kBKV;
    if (k0 + kBKV > kv_end) mask_tile(sA, k0, hf, kv_end);
  }
  float hsum = softmax_half(sA, 0);

  // Iteration jt: S(jt) is in sc with the probabilities of its pairs 0..7
  // already in pw and their per-lane sum in hsum.
  //   phase A: QK of tile jt+1 into sn  ||  pairs 8..15 of tile jt
  //   phase B: PV of tile jt            ||  pairs 0..7 of tile jt+1
  // The ring stage of tile jt is STAGE = jt % kNStage, a constant in each
  // of the loop's four bodies.
  auto iteration = [&](auto stage, int jt, f32x16 (&sc)[2], f32x16 (&sn)[2]) {
    constexpr int S = decltype(stage)::value;
    const bool has_next = jt + 1 < ntiles;
    // table reads first: their wait joins the tile wait below
    const int k_next = has_next ? tile_of(jt + 1) * kBKV : 0;
    const int t_issue = jt + kDist < ntiles ? tile_of(jt + kDist) : 0;
    {
      int pend = ntiles - 1 - (jt + 1);
      if (pend > kDist - 2) pend = kDist - 2;
      if (pend < 0) pend = 0;
      wait_tiles(pend);  // tile jt+1 resident; tile jt-1's stage is free
    }
    // Tile jt+kDist goes into the stage tile jt-2 used (free since the
    // barrier above), its DMA instructions spread over phase A's MFMAs:
    // part p beside MFMA floor((2p+1) NM / 2P).  Issued together after the
    // barrier, the workgroup's 32 queued at the CU's address unit, and the
    // wavefronts, issuing in order, waited behind theirs with their MFMAs
    // stalled.  Past the last tile the request is empty (no branch inside
    // the interleaved phase; the epilogue drains it).
    const TileReq req = tile_req(jt + kDist < ntiles, jt + kDist, t_issue);
    constexpr int NM = QK8 ? 4 : 2 * L::kSteps, NP = L::kLoadsPerTile;
    auto dma = [&](int i) {
#pragma unroll
      for (int part = 0; part < NP; ++part)
        if (i == (2 * part + 1) * NM / (2 * NP)) dma_part(req, part);
    };
    auto dma_b = no_dma;
    // second half of tile jt (first half already in pw, its sum in hsum)
    // (On the last tile the QK product runs on a stale or zero-filled LDS
    // stage and its scores are never used.  Selecting softmax_half there
    // instead let the compiler hoist the 16 exps shared by both arms above
    // the branch, out of the MFMA interleave.)
    float sum = hsum + phase_a(T{}, IC<(S + 1) % kNStage>{}, sn, sc, dma);
    const bool first = jt == 0 && !fixed;
    if (first || wave_any(!(sum <= trip)))
      sum = softmax_fixup(sc, sn, first, m, l, negm, pw, o, shift);
    l += sum;
    if (has_next && k_next + kBKV > kv_end) mask_tile(sn, k_next, hf, kv_end);
    // + pairs 0..7 of tile jt+1.  On the last tile this exponentiates the
    // stale contents of sn into pw words that nothing reads afterwards: one
    // phase-B body in the loop keeps its register allocation within the
    // 256 VGPRs of two wavefronts per SIMD (two bodies spilled).
    phase_b(T{}, IC<S>{}, sn, hsum, dma_b);
  };

  int jt = 0;
  static_assert(kNStage == 4, "the key loop is unrolled over the ring");
  for (; jt < ntiles; jt += 4) {
    iteration(IC<0>{}, jt, sA, sB);
    if (jt + 1 >= ntiles) break;
    iteration(IC<1>{}, jt + 1, sB, sA);
    if (jt + 2 >= ntiles) break;
    iteration(IC<2>{}, jt + 2, sA, sB);
    if (jt + 3 >= ntiles) break;
    iteration(IC<3>{}, jt + 3, sB, sA);
  }

  // the empty requests of the last iterations still write their stages
  // (zeros), one of them a stage the epilogue stages o through: drain every
  // wave's before any wave writes there
  wait_vmcnt(0);
  __syncthreads();

  // ---- epilogue: lane holds row q0 + l32, channels 32mb + 8g + 4hf + e
  const float ltot = l + __shfl_xor(l, 32, 64);
  const float unshift = fixed ? 1.0f : 1.0f / 16777216.0f;  // 2^-kPShift
  {
    const int row = q0 + l32;
    if (out32 != nullptr && hf == 0 && row < p.Sq) {
      const int64_t bhrow = out_row(row);
      // the residual (m, l) of the reference itself: kPShift taken out
      out_m[bhrow] = m + shift;
      out_l[bhrow] = ltot * unshift;
    }
  }
  // o goes out through LDS: in the accumulator layout a store instruction
  // writes 16 bytes (fp32: 32) into each of 32 rows, so a wave's rows take
  // 16 instructions touching 32 lines each.  Each wave instead writes its
  // rows, one pass of RB-byte row slices at a time, into a private 32 x RB
  // region of a ring stage the last iteration does not read (stages
  // (jl+2)%4 and (jl+3)%4; the drain above left no DMA pending), reads them back as
  // whole slices and stores 16 contiguous bytes per lane.  16-byte chunk j
  // of slice row r sits at chunk j ^ (r % (RB/16)).  bf16 K stages hold
  // two regions of RB = 2D bytes (bf16 o in one pass, fp32 o in two); with
  // E4M3 keys the regions are 128-byte slices in the two free V stages
  // (bf16 o in two passes, fp32 o in four).
  constexpr int RB = QK8 ? 128 : 2 * D;  // slice bytes per row
  constexpr int NCH = RB / 16;           // 16-byte chunks per slice
  constexpr int RPI = 64 / NCH;          // rows per read-back instruction
  constexpr int WPS = QK8 ? 4 : 2;       // wave regions per stage
  static_assert((QK8 ? L::kVTileB : L::kKTileB) >= WPS * 32 * RB &&
                    L::kVTileB >= WPS * 32 * RB,
                "a stage holds its wave regions");
  const int jl = ntiles - 1;
  const int grp = wave / WPS;  // QK8: V stages 0, 1; else K 0, 1, V 0, 1
  const int st = (jl + 2 + (grp & 1)) & 3;
  lds_u8* reg = lds + ((QK8 || grp >= 2) ? L::kVOff + st * L::kVTileB
                                         : st * L::kKTileB) +
                (wave % WPS) * (32 * RB);
  // (lane laundered through an empty asm: the compiler otherwise shares
  // these swizzled offsets with the key-operand offsets, computes them
  // before the key loop and spills them across it)
  int el = lane;
  asm volatile("" : "+v"(el));
  const int e32 = el & 31, ehf = el >> 5;
  const int ck = el % NCH;  // the lane's chunk in read-back
  auto slice_ptr = [&](int r) {  // read-back chunk of slice row r
    return (const __attribute__((address_space(3))) u32x4*)(
        reg + r * RB + ((ck ^ (r & (NCH - 1))) * 16));
  };
  if (out32 != nullptr) {
    constexpr int MPP = RB / 4 / 32;  // accumulator blocks per pass
#pragma unroll
    for (int ps = 0; ps < NB / MPP; ++ps) {
#pragma unroll
      for (int mh = 0; mh < MPP; ++mh)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          f32x4 w;
#pragma unroll
          for (int e = 0; e < 4; ++e)
            w[e] = o[ps * MPP + mh][g * 4 + e] * unshift;
          const int pc = (8 * mh + 2 * g + ehf) ^ (e32 & (NCH - 1));
          *(__attribute__((address_space(3))) f32x4*)(reg + e32 * RB + pc * 16) = w;
        }
#pragma unroll
      for (int i = 0; i < 32 / RPI; ++i) {
        const int r = i * RPI + el / NCH;
        const u32x4 v = *slice_ptr(r);
        if (q0 + r < p.Sq)
          *(u32x4*)(out32 + out_row(q0 + r) * D + ps * (RB / 4) + 4 * ck) = v;
      }
    }
  }
  if (out_o != nullptr) {
    constexpr int MPP = RB / 2 / 32;
    const float inv = 1.0f / ltot;
    uint16_t* obase = out_o + b * p.o_sb + h * p.o_sh;
    // the ABI guarantees 8-byte aligned rows; 16-byte stores where the
    // tensor and its strides allow them (a uniform branch)
    const bool al16 = (((uintptr_t)p.o & 15u) | ((p.o_sb | p.o_sh | p.o_ss) & 7)) == 0;
#pragma unroll
    for (int ps = 0; ps < NB / MPP; ++ps) {
#pragma unroll
      for (int mh = 0; mh < MPP; ++mh)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const f32x16& om = o[ps * MPP + mh];
          u32x2 w;
          w[0] = pack_bf16x2(om[g * 4 + 0] * inv, om[g * 4 + 1] * inv);
          w[1] = pack_bf16x2(om[g * 4 + 2] * inv, om[g * 4 + 3] * inv);
          const int pc = (4 * mh + g) ^ (e32 & (NCH - 1));
          *(__attribute__((address_space(3))) u32x2*)(reg + e32 * RB + pc * 16 +
                                                       8 * ehf) = w;
        }
#pragma unroll
      for (int i = 0; i < 32 / RPI; ++i) {
        const int r = i * RPI + el / NCH;
        const u32x4 v = *slice_ptr(r);
        if (q0 + r < p.Sq) {
          uint16_t* dst = obase + (int64_t)(q0 + r) * p.o_ss + ps * (RB / 2) + 8 * ck;
          if (al16) {
            *(u32x4*)dst = v;
          } else {
            *(u32x2*)dst = u32x2{v[0], v[1]};
            *(u32x2*)(dst + 4) = u32x2{v[2], v[3]};
          }
        }
      }
    }
  }
}

// Combines the n_split parts of every split query block (the tail split):
// with M the largest m of the parts that saw keys (l > 0), weights
// w = exp2(m - M), l = sum w*l_part and o = sum w*o_part, in LSE space as
// kernels/splash.py:653-662 merges residuals; then writes the normalized
// o and/or the residual (o, M, l) exactly where the unsplit kernel would.
// D/4 lanes per row, 4 channels each; 256 / (D/4) rows per 256-thread block.
// NS bounds n_split (2, 4, 8 or 16): every part's loads are in flight at
// once, and a small bound keeps the register count, and so the occupancy
// that hides HBM latency, where the split is narrow.
template <int D, int NS>
__global__ __launch_bounds__(256) void split_merge_kernel(FlashParams p) {
  constexpr int LPR = D / 4, RPB = 256 / LPR;
  const int g = blockIdx.x * RPB + (threadIdx.x / LPR);
  const int c = 4 * (threadIdx.x % LPR);
  const int tq = g / kBQ, r = g - tq * kBQ;
  if (tq >= p.n_tail) return;
  const int wg = p.n_main + tq;
  const int qblk = wg % p.n_qblk;
  const int bh = wg / p.n_qblk;
  const int h = bh % p.Hq;
  const int b = bh / p.Hq;
  const int row = qblk * kBQ + r;
  if (row >= p.Sq) return;
  const int64_t units = (int64_t)p.n_tail * p.n_split;
  const float* wm = p.ws + units * kBQ * D;
  const float* wl = wm + units * kBQ;
  const int64_t r0 = (int64_t)tq * p.n_split * kBQ + r;  // part 0's row
  // Every part's m, l and o slice is requested before any is used (the
  // loop runs to NS under a uniform branch per part), so the merge pays
  // one memory latency instead of one per part.
  const int last = p.n_split - 1;
  float ms[NS], ls[NS];
  f32x4 os[NS];
#pragma unroll
  for (int i = 0; i < NS; ++i) {
    ms[i] = 0.f;
    ls[i] = 0.f;
    os[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    if (i <= last) {
      const int64_t ri = r0 + (int64_t)i * kBQ;
      ms[i] = wm[ri];
      ls[i] = wl[ri];
      os[i] = *(const f32x4*)(p.ws + ri * D + c);
    }
  }
  float mx = -INFINITY;
#pragma unroll
  for (int i = 0; i < NS; ++i)
    if (i <= last && ls[i] > 0.f) mx = fmaxf(mx, ms[i]);
  float lsum = 0.f;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < NS; ++i) {
    const float w = (i <= last && ls[i] > 0.f) ? exp2f(ms[i] - mx) : 0.f;
    lsum += w * ls[i];
#pragma unroll
    for (int e = 0; e < 4; ++e) acc[e] += w * os[i][e];
  }
  const int64_t bhrow = ((int64_t)b * p.Hq + h) * p.Sq + row;
  if (p.o32 != nullptr) {
    *(f32x4*)(p.o32 + bhrow * D + c) = acc;
    if (c == 0) {
      p.m[bhrow] = lsum > 0.f ? mx : 0.f;
      p.l[bhrow] = lsum;
    }
  }
  if (p.o != nullptr) {
    const float inv = lsum > 0.f ? 1.0f / lsum : 0.f;
    u32x2 w;
    w[0] = pack_bf16x2(acc[0] * inv, acc[1] * inv);
    w[1] = pack_bf16x2(acc[2] * inv, acc[3] * inv);
    *(u32x2*)(p.o + b * p.o_sb + h * p.o_sh + (int64_t)row * p.o_ss + c) = w;
  }
}

template <int D, bool QK8, bool SPARSE, bool VT>
static int launch_flash(const FlashParams& base, hipStream_t st) {
  using L = Stage<D, QK8>;
  FlashParams p = base;
  p.n_qblk = (p.Sq + kBQ - 1) / kBQ;
  const int64_t nwg = (int64_t)p.n_qblk * p.Hq * p.B;
  if (nwg > 0x7fffffff)
    return set_error(DT_ERR_SHAPE, "dt_flash_fwd: grid too large");
  // per-(b, head) K/V ranges are addressed with 32-bit buffer offsets
  if ((int64_t)p.kv_end * p.k_ss * (QK8 ? 1 : 2) >= (1ll << 32) ||
      (!VT && (int64_t)p.kv_end * p.v_ss * 2 >= (1ll << 32)))
    return set_error(DT_ERR_UNSUPPORTED,
                     "dt_flash_fwd: K/V slice of one head exceeds 4 GiB");
  p.n_wg = (int)nwg;
  if (p.n_split > kMaxSplit)  // the planner stays within it; the merge relies on it
    return set_error(DT_ERR_ARG, "dt_flash_fwd: %d split parts > %d",
                     p.n_split, kMaxSplit);
  if (p.ws == nullptr || p.n_split <= 1) {
    p.n_split = 1;
    p.n_tail = 0;
    p.n_main = p.n_wg;
  }
  const void* fn = (const void*)flash_attn_kernel<D, QK8, SPARSE, VT>;
  static std::atomic<uint64_t> lds_set{0};
  if (int rc = ensure_lds_limit(fn, L::kLds, lds_set, "dt_flash_fwd"))
    return rc;
  const int grid = p.n_main + p.n_tail * p.n_split;
  hipLaunchKernelGGL((flash_attn_kernel<D, QK8, SPARSE, VT>), dim3(grid),
                     dim3(kNW * 64), L::kLds, st, p);
  if (p.n_tail > 0) {
    const dim3 mg(p.n_tail * (kBQ / (256 / (D / 4))));
    if (p.n_split <= 2)
      hipLaunchKernelGGL((split_merge_kernel<D, 2>), mg, dim3(256), 0, st, p);
    else if (p.n_split <= 4)
      hipLaunchKernelGGL((split_merge_kernel<D, 4>), mg, dim3(256), 0, st, p);
    else if (p.n_split <= 8)
      hipLaunchKernelGGL((split_merge_kernel<D, 8>), mg, dim3(256), 0, st, p);
    else
      hipLaunchKernelGGL((split_merge_kernel<D, kMaxSplit>), mg, dim3(256), 0,
                         st, p);
  }
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return set_error(DT_ERR_LAUNCH, "dt_flash_fwd: %s", hipGetErrorString(e));
  return DT_OK;
}

SplitPlan split_plan(int64_t n_wg, int ntiles, int n_cu, int D, size_t max_ws) {
  SplitPlan sp{1, 0, (int)n_wg, 0};
  if (n_cu <= 0 || n_wg <= 0) return sp;
  const int64_t rem = n_wg % n_cu;
  if (rem == 0) return sp;
  // The last round's rem query blocks cut into ns parts run as
  // ceil(rem * ns / n_cu) rounds of parts of ntiles / ns tiles; each
  // workgroup also pays a start-up (q load, the first tiles' latency, the
  // epilogue) of about kStartTiles tiles, and the merge reads every part
  // (about kMergeTiles per part).  Pick the ns (at most 16, at least two
  // tiles per part, workspace at most max_ws and 512 MiB) with the shortest
  // tail.
  constexpr int64_t kStartTiles = 8;  // fitted: I1 with 5 parts ran 3.8 % slower than with 2
  constexpr int64_t kMergeTiles = 1;  // fitted: P (16 tiles) 17.4 us at 4 parts, 19.8 at 8
  constexpr size_t kMaxWs = size_t(512) << 20;
  if (max_ws > kMaxWs) max_ws = kMaxWs;
  const size_t unit_bytes = (size_t)kBQ * (D + 2) * sizeof(float);
  int64_t best_ns = 1, best_cost = ntiles + kStartTiles;
  for (int64_t ns = 2; ns <= kMaxSplit && ns <= ntiles / 2; ++ns) {
    if ((size_t)(rem * ns) * unit_bytes > max_ws) break;
    const int64_t rounds = (rem * ns + n_cu - 1) / n_cu;
    const int64_t cost =
        rounds * ((ntiles + ns - 1) / ns + kStartTiles) + ns * kMergeTiles;
    if (cost < best_cost) {
      best_cost = cost;
      best_ns = ns;
    }
  }
  if (best_ns < 2) return sp;
  sp.n_split = (int)best_ns;
  sp.n_tail = (int)rem;
  sp.n_main = (int)(n_wg - rem);
  sp.ws_bytes = (size_t)(rem * best_ns) * unit_bytes;
  return sp;
}

// The CU count of the current device, queried once per device (every
// planned call asks for it).
int device_cu_count(int* n_cu) {
  constexpr int kMaxDev = 64;
  static std::atomic<int> cache[kMaxDev];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess)
    return set_error(DT_ERR_LAUNCH, "dt_flash_fwd: no current device");
  if (dev >= 0 && dev < kMaxDev) {
    const int c = cache[dev].load(std::memory_order_relaxed);
    if (c > 0) {
      *n_cu = c;
      return DT_OK;
    }
  }
  if (hipDeviceGetAttribute(n_cu, hipDeviceAttributeMultiprocessorCount,
                            dev) != hipSuccess)
    return set_error(DT_ERR_LAUNCH, "dt_flash_fwd: CU count query failed");
  if (dev >= 0 && dev < kMaxDev && *n_cu > 0)
    cache[dev].store(*n_cu, std::memory_order_relaxed);
  return DT_OK;
}

template <bool QK8, bool SPARSE>
static int launch_d128_v(const FlashParams& p, hipStream_t st) {
  return p.vt != nullptr ? launch_flash<128, QK8, SPARSE, true>(p, st)
                         : launch_flash<128, QK8, SPARSE, false>(p, st);
}

int launch_flash_attn(const FlashParams& p, int D, hipStream_t st) {
  if (D == 64) {
    if (p.k8 != nullptr || p.vt != nullptr || p.tile_span != nullptr)
      return set_error(DT_ERR_UNSUPPORTED,
                       "dt_flash_fwd: head dim 64 takes bf16 keys, row-major "
                       "V and no tile table");
    return launch_flash<64, false, false, false>(p, st);
  }
  const bool sparse = p.tile_span != nullptr;
  if (p.k8 != nullptr)
    return sparse ? launch_d128_v<true, true>(p, st)
                  : launch_d128_v<true, false>(p, st);
  return sparse ? launch_d128_v<false, true>(p, st)
                : launch_d128_v<false, false>(p, st);
}

}  // namespace dt
