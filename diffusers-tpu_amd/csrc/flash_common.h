// Definitions shared by the flash-attention kernels (gfx950).
#pragma once

#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include <atomic>

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
  const float* mk;  // fixed-m operand [2][Hq] or null
  const int32_t* kv_len_dev;
  int kv_len_count;  // entries of kv_len_dev: <= 1 shared, else one per b
  const uint8_t* k8;  // E4M3 keys (qk_fp8) instead of k, or null
  // block-sparse table or nulls: per (query head, 256-row query block) a
  // [begin, end) span of tile_ids, the 64-key tiles to visit
  const int32_t* tile_span;
  const int32_t* tile_ids;
  // packed V (dt_pack_v layout) instead of v, or null: per (b, kv head)
  // vt_tiles tiles of 64 keys, each a contiguous [128][64] bf16 block
  // (channel-major, keys permuted within 16-key groups to the score
  // accumulator's order), zero past kv_end
  const uint16_t* vt;
  int64_t vt_tiles;
  // Tail split (D = 64 and 128): workgroups [0, n_main) each run one query
  // block over all its keys; the n_tail query blocks after them run as
  // n_split parts each, one per workgroup, every part a contiguous share of
  // the block's key tiles, writing unnormalized o, m, l for its 256 rows to
  // ws (o: [units][256][128], then m and l: [units][256] each, units =
  // n_tail * n_split); a merge kernel combines the parts.  n_split = 1 and
  // n_tail = 0 when there is no split.
  float* ws;
  int n_main, n_split, n_tail;
  int64_t q_sb, q_sh, q_ss;
  int64_t k_sb, k_sh, k_ss;
  int64_t v_sb, v_sh, v_ss;
  int64_t o_sb, o_sh, o_ss;
  int B, Hq, Hkv, Sq, Skv;
  int kv_end;      // keys [0, kv_end) take part (upper bound if kv_len_dev)
  // runtime key length in device memory, or null: the kernels then run with
  // resolve_len(kv_len_dev, kv_len_count, b, kv_end, Skv) keys instead of
  // kv_end
  int n_qblk;      // query blocks per (b, h)
  int n_wg;        // workgroups in the grid
  float c;         // scale * log2(e)
};

typedef short v4i16 __attribute__((ext_vector_type(4)));
typedef short v8i16 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) uint8_t lds_u8;

__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  // v_cvt_pk_bf16_f32 (round to nearest even)
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  bf16x2 r = {(__bf16)a, (__bf16)b};
  return *reinterpret_cast<uint32_t*>(&r);
}

// Workgroup remap: workgroups are dealt round-robin to the 8 XCDs; give XCD
// x (= blockIdx % 8) a contiguous range of logical workgroups so that the
// query blocks sweeping the same keys share that XCD's L2.
__device__ __forceinline__ int xcd_remap(int bid, int n) {
  const int xcd = bid & 7, idx = bid >> 3;
  const int per = n >> 3, rem = n & 7;
  return (xcd < rem) ? xcd * (per + 1) + idx
                     : rem * (per + 1) + (xcd - rem) * per + idx;
}

// 16 bytes per lane, global -> LDS through a buffer descriptor
// (buffer_load_dwordx4 ... lds): lane i's 16 bytes, read at byte offset
// voff of the buffer, land at LDS byte address lds_base + 16*i.  Offsets at
// or past the descriptor's num_records read as zeros.  Issued as inline
// assembly so that the compiler does not treat every later LDS read as
// possibly aliasing it (it would otherwise wait for all outstanding tile
// loads before each LDS read, defeating the prefetch).  Completion is the
// caller's job: wait on vmcnt, then barrier, before reading the tile.
// m0 is listed as clobbered.  The compiler warns that it does not preserve
// reserved registers across the statement.  That is safe for the kernels
// that call it: they use no other m0-based instruction (no indexed register
// moves, no GWS or message ops; in the gfx950 assembly every m0 write is
// this helper's, each followed by its load), and gfx9-family LDS
// instructions do not read m0, so no value of the compiler's lives in m0.
__device__ __forceinline__ void lds_dma16_buf(u32x4 rsrc, uint32_t voff,
                                              uint32_t lds_base) {
  asm volatile(
      "s_mov_b32 m0, %2\n\t"
      "buffer_load_dwordx4 %0, %1, 0 offen lds"
      :
      : "v"(voff), "s"(rsrc), "s"(lds_base)
      : "memory", "m0");
}

// Raw buffer descriptor over [base, base + bytes) (stride 0; the dword3
// format word makes untyped dword loads valid on gfx9-family parts).
__device__ __forceinline__ u32x4 make_rsrc(uint64_t base, uint32_t bytes) {
  u32x4 r;
  r[0] = (uint32_t)base;
  r[1] = (uint32_t)(base >> 32) & 0xffffu;
  r[2] = bytes;
  r[3] = 0x00020000u;
  return r;
}

// s_waitcnt with only the vector-memory count constrained (n in 0..15;
// larger n waits for everything).
__device__ __forceinline__ void wait_vmcnt(int n) {
  // vmcnt[3:0] in bits 3:0 (vmcnt[5:4] in bits 15:14 stay 0); expcnt and
  // lgkmcnt left at their maxima (no constraint).
#define DT_VMCNT_CASE(k) \
  case k: __builtin_amdgcn_s_waitcnt(0x0F70 | k); break;
  switch (n) {
    DT_VMCNT_CASE(1) DT_VMCNT_CASE(2) DT_VMCNT_CASE(3) DT_VMCNT_CASE(4)
    DT_VMCNT_CASE(5) DT_VMCNT_CASE(6) DT_VMCNT_CASE(7) DT_VMCNT_CASE(8)
    DT_VMCNT_CASE(9) DT_VMCNT_CASE(10) DT_VMCNT_CASE(11) DT_VMCNT_CASE(12)
    DT_VMCNT_CASE(13) DT_VMCNT_CASE(14) DT_VMCNT_CASE(15)
    default: __builtin_amdgcn_s_waitcnt(0x0F70); break;
  }
#undef DT_VMCNT_CASE
}

// s_waitcnt on the vector-memory count alone, for a compile-time count up
// to 63 (vmcnt[3:0] in bits 3:0, vmcnt[5:4] in bits 15:14).
template <int N>
__device__ __forceinline__ void wait_vmcnt_c() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 15) | ((N >> 4) << 14));
}

typedef int i32x8 __attribute__((ext_vector_type(8)));

// Four bf16 values (two packed words, low half first) -> four E4M3 bytes
// (OCP e4m3fn), clamped to +-448 first as quantize_saturating does
// (kernels/fp8_cast.py:28-39); v_cvt_pk_fp8_f32 rounds to nearest even.
__device__ __forceinline__ int pack_e4m3x4(uint32_t w0, uint32_t w1) {
  auto sat = [](uint32_t bits) {
    return fminf(fmaxf(__uint_as_float(bits), -448.0f), 448.0f);
  };
  int r = __builtin_amdgcn_cvt_pk_fp8_f32(sat(w0 << 16), sat(w0 & 0xffff0000u),
                                          0, false);
  return __builtin_amdgcn_cvt_pk_fp8_f32(sat(w1 << 16), sat(w1 & 0xffff0000u), r,
                                         true);
}

__device__ __forceinline__ bool wave_any(bool x) {
  return __builtin_amdgcn_ballot_w64(x) != 0;
}

// Raises a kernel's dynamic-LDS limit to `bytes`, once per device (the
// attribute belongs to the device that is current when it is set).  `done`
// is a per-kernel bitmask of devices already set up.
inline int ensure_lds_limit(const void* fn, int bytes,
                            std::atomic<uint64_t>& done, const char* who) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess)
    return set_error(DT_ERR_LAUNCH, "%s: no current device", who);
  const uint64_t bit = dev < 64 ? (1ull << dev) : 0;
  if (bit && (done.load(std::memory_order_acquire) & bit)) return DT_OK;
  const hipError_t e = hipFuncSetAttribute(
      fn, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  if (e != hipSuccess)
    return set_error(DT_ERR_LAUNCH, "%s: LDS limit %d B: %s", who, bytes,
                     hipGetErrorString(e));
  done.fetch_or(bit, std::memory_order_release);
  return DT_OK;
}

// Launcher (flash_attn.hip): head dim D = 64 or 128.
int launch_flash_attn(const FlashParams& p, int D, hipStream_t st);
// Launcher (flash_wide.hip): head dim 256, bf16 keys, row-major V, no tile
// table, no tail split.
int launch_flash_wide(const FlashParams& p, hipStream_t st);

// Tail split plan for a launch of n_wg workgroups over ntiles key
// tiles on a device of n_cu compute units (one workgroup per CU): the
// number of parts the last, partly filled round's query blocks are cut
// into (1: no split), and the workspace bytes it needs, at most max_ws
// (fewer parts when the best plan needs more).
struct SplitPlan {
  int n_split, n_tail, n_main;
  size_t ws_bytes;
};
SplitPlan split_plan(int64_t n_wg, int ntiles, int n_cu, int D,
                     size_t max_ws = ~size_t(0));
int device_cu_count(int* n_cu);

}  // namespace dt
