// C ABI of the non-causal flash attention forward (gfx950): argument
// checks, the parameter block, the tail-split plan and the launch of
// flash_attn_kernel (flash_attn.hip, head dims 64 and 128).
//
// Replaces the reference's splash entry points: kernels/splash.py:566-650
// (`attention`) and the residual form :665-742, with the kernel body
// _flash_attention_kernel :115-375 in flash_attn.hip.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include <mutex>

#include "../../include/dt_attention.h"
#include "dt_common.h"
#include "flash_common.h"

namespace dt {

static bool al16(const void* ptr) { return ((uintptr_t)ptr & 15u) == 0; }

}  // namespace dt

namespace dt {
namespace {

// The tail-split plan of a launch of B * Hq * ceil(Sq / 256) query blocks
// over kv_end keys on the current device, within ws_bytes of workspace;
// dt_flash_fwd_ex, dt_flash_fwd_workspace_bytes and dt_flash_fwd_plan all
// plan through here.
int plan_launch(int B, int Hq, int Sq, int kv_end, int D, size_t ws_bytes,
                int* n_cu, SplitPlan* sp) {
  if (int rc = device_cu_count(n_cu)) return rc;
  const int64_t n_wg = (int64_t)B * Hq * ((Sq + 255) / 256);
  *sp = split_plan(n_wg, (kv_end + 63) / 64, *n_cu, D, ws_bytes);
  return DT_OK;
}

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
  if (D != 64 && D != 128 && D != 256)
    return set_error(DT_ERR_UNSUPPORTED,
                     "dt_flash_fwd: head dim %d (supported: 64, 128, 256)", D);
  if (D == 256 && (k_e4m3 || packed || tile_span != nullptr))
    return set_error(DT_ERR_UNSUPPORTED,
                     "dt_flash_fwd: head dim 256 takes bf16 keys, row-major V "
                     "and no tile table");
  // With the length in device memory the host plans for every key: the
  // grid, the packed-V tile count and the split cover Skv, and the kernels
  // skip the tiles past the length they read.  kv_len is then the number of
  // entries kv_len_dev holds (one for the batch, or B).
  int kv_len_count = 0;
  if (int rc = dev_len_count(kv_len_dev, kv_len, B, "dt_flash_fwd",
                             &kv_len_count))
    return rc;
  if (kv_len_dev != nullptr) kv_len = 0;
  if (kv_len > Skv)
    return set_error(DT_ERR_SHAPE, "dt_flash_fwd: kv_len %d > Skv %d", kv_len, Skv);
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
  p.kv_len_count = kv_len_count;
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
  // (head dim 256 runs unsplit: the workspace is not used)
  if (ws != nullptr && D != 256) {
    if (!al16(ws))
      return set_error(DT_ERR_UNSUPPORTED, "dt_flash_fwd_ex: misaligned workspace");
    int n_cu = 0;
    SplitPlan sp;
    if (int rc = plan_launch(B, Hq, Sq, p.kv_end, D, ws_bytes, &n_cu, &sp))
      return rc;
    if (sp.n_split > 1 && sp.ws_bytes <= ws_bytes) {
      p.ws = (float*)ws;
      p.n_split = sp.n_split;
      p.n_tail = sp.n_tail;
      p.n_main = sp.n_main;
    }
  }
  if (D == 256) return launch_flash_wide(p, st);
  return launch_flash_attn(p, D, st);
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
  if ((D != 64 && D != 128) || B <= 0 || Hq <= 0 || Sq <= 0 || Skv <= 0)
    return 0;
  const int kv_end = (kv_len <= 0 || kv_len > Skv) ? Skv : kv_len;
  int n_cu = 0;
  dt::SplitPlan sp;
  if (dt::plan_launch(B, Hq, Sq, kv_end, D, ~size_t(0), &n_cu, &sp) != DT_OK)
    return 0;
  return sp.ws_bytes;
}

extern "C" int dt_flash_fwd_plan(int B, int Hq, int Sq, int Skv, int kv_len,
                                 int D, size_t workspace_bytes, int32_t* plan,
                                 size_t* ws_needed) {
  if (plan == nullptr || ws_needed == nullptr)
    return dt::set_error(DT_ERR_ARG, "dt_flash_fwd_plan: null output");
  if (D != 64 && D != 128 && D != 256)
    return dt::set_error(DT_ERR_UNSUPPORTED,
                         "dt_flash_fwd_plan: head dim %d (supported: 64, 128, "
                         "256)", D);
  if (B <= 0 || Hq <= 0 || Sq <= 0 || Skv <= 0 || kv_len > Skv)
    return dt::set_error(DT_ERR_SHAPE, "dt_flash_fwd_plan: bad shape");
  const int kv_end = (kv_len <= 0) ? Skv : kv_len;
  if (D == 256) {  // 128-row blocks over 32-key tiles, never split
    int n_cu = 0;
    if (int rc = dt::device_cu_count(&n_cu)) return rc;
    const int64_t n_wg = (int64_t)B * Hq * ((Sq + 127) / 128);
    plan[0] = n_cu;
    plan[1] = (int32_t)n_wg;
    plan[2] = (kv_end + 31) / 32;
    plan[3] = 1;
    plan[4] = 0;
    plan[5] = (int32_t)n_wg;
    *ws_needed = 0;
    return DT_OK;
  }
  int n_cu = 0;
  dt::SplitPlan sp;
  if (int rc = dt::plan_launch(B, Hq, Sq, kv_end, D, workspace_bytes, &n_cu, &sp))
    return rc;
  const bool split = sp.n_split > 1 && sp.ws_bytes <= workspace_bytes;
  const int64_t n_wg = (int64_t)B * Hq * ((Sq + 255) / 256);
  plan[0] = n_cu;
  plan[1] = (int32_t)n_wg;
  plan[2] = (kv_end + 63) / 64;
  plan[3] = split ? sp.n_split : 1;
  plan[4] = split ? sp.n_tail : 0;
  plan[5] = split ? sp.n_main : (int32_t)n_wg;
  *ws_needed = split ? sp.ws_bytes : 0;
  return DT_OK;
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
