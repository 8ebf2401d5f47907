// Packed-V layout for the D = 128 attention kernel (gfx950).
//
// The attention kernel's PV product takes V^T as its MFMA A operand: a lane
// holds 8 keys of one channel.  Row-major V gives those through the
// transposing LDS read ds_read_b64_tr_b16, two per operand; this pass stores
// V channel-major instead, so that the operand is one ds_read_b128, at about
// twice the LDS bytes per clock.
//
// Layout, per (b, kv head): `tiles` blocks of 64 keys, each one contiguous
// [128][64] bf16 matrix (16 KiB) whose row d holds channel d of the
// tile's keys, so a tile is one 16 KiB read like a row-major V tile (a
// channel-major row spanning the whole sequence put a tile's 128 rows far
// apart in memory and doubled the attention kernel's fetches past L2).
// Within each group of 16 keys, column j holds key
// perm(j) = (j & 3) | ((j & 4) << 1) | ((j & 8) >> 1), i.e. keys
// 0-3, 8-11, 4-7, 12-15: the order in which a score-accumulator lane half
// holds its keys, so that 8 consecutive columns are exactly the 8 keys of
// one probability operand.  Keys from kv_end to the end of the last tile
// are zero.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/dt_attention.h"
#include "flash_common.h"

namespace dt {
namespace {

struct PackParams {
  const uint16_t* v;
  uint16_t* vt;
  int64_t v_sb, v_sh, v_ss;
  int64_t tiles;
  int Hkv, kv_end, Skv;
  const int32_t* kv_len_dev;  // runtime key length, or null (kv_end)
  int kv_len_count;           // its entries: <= 1 shared, else one per b
};

constexpr int kPackKeys = 64;
constexpr int kPackPad = 8;  // LDS row padding (elements)

// 16-byte chunk of key row `key` that holds channels 8*ch .. 8*ch+7.  A
// wavefront's transposing reads take one channel from 8 keys spread over
// rows r, r+16, r+32, r+48 (and r+4 ...); with 272-byte rows the 16-row
// steps land in the same LDS bank, so the chunk is XOR-ed with the row's
// 16-row group, which puts those reads in four different banks.
__device__ __forceinline__ int swz(int key, int ch) {
  return ch ^ ((key >> 4) & 3);
}

__global__ __launch_bounds__(256) void v_pack_kernel(PackParams p) {
  __shared__ __attribute__((aligned(16))) uint16_t t[kPackKeys][128 + kPackPad];
  const int tid = threadIdx.x;
  const int kv0 = blockIdx.x * kPackKeys;
  const int h = blockIdx.y % p.Hkv;
  const int b = blockIdx.y / p.Hkv;
  const int kv_end = resolve_len(p.kv_len_dev, p.kv_len_count, b, p.kv_end, p.Skv);
  if (kv0 >= kv_end) return;  // a tile past a runtime length: never read
  const uint16_t* src = p.v + b * p.v_sb + h * p.v_sh;
#pragma unroll
  for (int it = 0; it < 4; ++it) {
    const int idx = it * 256 + tid;
    const int key = idx >> 4, ch = idx & 15;
    u32x4 x = {0u, 0u, 0u, 0u};
    if (kv0 + key < kv_end)
      x = __builtin_nontemporal_load(
          (const u32x4*)(src + (int64_t)(kv0 + key) * p.v_ss + ch * 8));
    *(u32x4*)&t[key][swz(key, ch) * 8] = x;
  }
  __syncthreads();
  uint16_t* dst = p.vt + ((int64_t)blockIdx.y * p.tiles + blockIdx.x) * (128 * kPackKeys);
#pragma unroll
  for (int it = 0; it < 4; ++it) {
    const int idx = it * 256 + tid;
    const int d = idx >> 3, c = idx & 7;
    uint32_t w[4];
#pragma unroll
    for (int e = 0; e < 8; e += 2) {
      const int j0 = 8 * (c & 1) + e, j1 = j0 + 1;
      const int k0 = 16 * (c >> 1) + ((j0 & 3) | ((j0 & 4) << 1) | ((j0 & 8) >> 1));
      const int k1 = 16 * (c >> 1) + ((j1 & 3) | ((j1 & 4) << 1) | ((j1 & 8) >> 1));
      w[e / 2] = (uint32_t)t[k0][swz(k0, d >> 3) * 8 + (d & 7)] |
                 ((uint32_t)t[k1][swz(k1, d >> 3) * 8 + (d & 7)] << 16);
    }
    const u32x4 o = {w[0], w[1], w[2], w[3]};
    __builtin_nontemporal_store(o, (u32x4*)(dst + d * kPackKeys + 8 * c));
  }
}

}  // namespace
}  // namespace dt

extern "C" int dt_pack_v(const uint16_t* v, uint16_t* vt, int B, int Hkv,
                         int Skv, int D, const int64_t* v_strides, int kv_len,
                         const int32_t* kv_len_dev, int64_t vt_tiles,
                         void* stream) {
  using namespace dt;
  if (!v || !vt || !v_strides)
    return set_error(DT_ERR_ARG, "dt_pack_v: null pointer argument");
  if (B <= 0 || Hkv <= 0 || Skv <= 0)
    return set_error(DT_ERR_SHAPE, "dt_pack_v: B=%d Hkv=%d Skv=%d", B, Hkv, Skv);
  if (D != 128)
    return set_error(DT_ERR_UNSUPPORTED, "dt_pack_v: head dim %d (supported: 128)",
                     D);
  // a length in device memory: plan every tile, the kernel skips the rest;
  // kv_len is then the entry count of kv_len_dev
  int kv_len_count = 0;
  if (int rc = dev_len_count(kv_len_dev, kv_len, B, "dt_pack_v", &kv_len_count))
    return rc;
  if (kv_len_dev != nullptr) kv_len = 0;
  if (kv_len > Skv)
    return set_error(DT_ERR_SHAPE, "dt_pack_v: kv_len %d > Skv %d", kv_len, Skv);
  const int kv_end = (kv_len > 0 && kv_len_dev == nullptr) ? kv_len : Skv;
  const int64_t need = (int64_t)(kv_end + 63) / 64;
  if (vt_tiles < need)
    return set_error(DT_ERR_SHAPE, "dt_pack_v: vt_tiles %lld < %lld key tiles",
                     (long long)vt_tiles, (long long)need);
  for (int i = 0; i < 3; ++i)
    if (v_strides[i] % 8)
      return set_error(DT_ERR_UNSUPPORTED,
                       "dt_pack_v: strides must be multiples of 8 elements");
  if (((uintptr_t)v & 15u) || ((uintptr_t)vt & 15u))
    return set_error(DT_ERR_UNSUPPORTED, "dt_pack_v: misaligned tensor");
  if ((int64_t)B * Hkv > 65535)
    return set_error(DT_ERR_SHAPE, "dt_pack_v: B*Hkv %lld too large",
                     (long long)B * Hkv);
  PackParams p;
  p.v = v;
  p.vt = vt;
  p.v_sb = v_strides[0];
  p.v_sh = v_strides[1];
  p.v_ss = v_strides[2];
  p.tiles = vt_tiles;
  p.Hkv = Hkv;
  p.kv_end = kv_end;
  p.Skv = Skv;
  p.kv_len_dev = kv_len_dev;
  p.kv_len_count = kv_len_count;
  hipLaunchKernelGGL(v_pack_kernel, dim3((unsigned)need, B * Hkv),
                     dim3(256), 0, (hipStream_t)stream, p);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return set_error(DT_ERR_LAUNCH, "dt_pack_v: %s", hipGetErrorString(e));
  return DT_OK;
}
