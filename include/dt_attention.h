/*
 * dt_attention.h — C ABI of the MI355X (gfx950) DiT attention hot path.
 *
 * Stream-ordered entry points that replace the two stages of the
 * reference's attention path (shungcp/diffusers-tpu), the prologue and the
 * attention call, and the helpers around them:
 *
 *   dt_qk_norm_rope  — QK-RMSNorm + RoPE (+ optional per-head q factor,
 *                      padded-row zeroing, layout change) in one pass.
 *                      Replaces the per-layer prologue
 *                      models/minimax_h3/jax_dit.py:362-381 (norm_q/norm_k
 *                      :362-363, apply_rope :365-366 defined :251-262,
 *                      padded-row zeroing :367-381), the same stage in
 *                      models/qwen_image_21/jax_dit.py:250-254 and
 *                      models/moss_image/jax_dit.py:173-176.
 *   dt_qk_norm_rope_f32 — the same with fp32 q and k.
 *   dt_qk_norm_rope_table — the same with the rotation's cos/sin read from
 *                      tables, as the reference's models pass them
 *                      (jax_dit.py:251-262 cos/sin; moss_image/jax_dit.py:
 *                      136-142 sin|cos rows); _f32: fp32 q and k.
 *   dt_flash_fwd     — non-causal flash attention forward with a runtime
 *                      key length.  Replaces kernels/splash.py:566-650
 *                      (`attention`, normalized output) and, with
 *                      `residual` outputs, kernels/splash.py:665-742
 *                      (`residual_attention`: unnormalized o, m, l); with
 *                      `mk`, the fixed-m softmax (kernels/splash.py:170-248).
 *   dt_max_row_norm  — per-head max L2 row norm, the reduction behind the
 *                      fixed-m bound (kernels/fixed_m_bound.py:57-118).
 *   dt_flash_fwd_qk8 — dt_flash_fwd with E4M3 keys and E4M3 scaled queries
 *                      in the QK product (qk_fp8, kernels/splash.py:420-424).
 *   dt_quantize_e4m3 — saturating bf16 -> E4M3 cast
 *                      (kernels/fp8_cast.py:28-39).
 *   dt_flash_fwd_blocksparse — dt_flash_fwd / _qk8 visiting, per query
 *                      block, a table of key tiles
 *                      (kernels/sparse_splash.py:568-662).
 *   dt_pack_v        — V into the channel-major "packed V" layout.
 *   dt_flash_fwd_ex  — dt_flash_fwd / _qk8 / _blocksparse in one, V
 *                      row-major or packed, optional tail-split workspace.
 *   dt_flash_fwd_workspace_bytes — the workspace dt_flash_fwd_ex can use.
 *   dt_flash_fwd_plan — the launch plan (grid, tail split) of a shape.
 *   dt_flash_fwd_ex_noalloc — dt_flash_fwd_ex with its workspace in static
 *                      device memory (no reference counterpart: for
 *                      callers that cannot allocate).
 *   dt_smooth_keys   — k - mean_S(k) with padded rows zeroed, and the
 *                      smoothed keys' per-head max row norm (the fixed-m
 *                      caller contract, models/minimax_h3/jax_server.py:
 *                      271-289).
 *   dt_fixed_m_prepare — the fixed-m operand of one call, with or without
 *                      the key smoothing, in three launches
 *                      (kernels/fixed_m_bound.py:98-118, splash.py:609-614).
 *
 * Conventions shared by every entry point:
 *   - Tensors are bf16 bit patterns (uint16_t) in device memory; the last
 *     (head-dim) axis is contiguous; other axes are given by element strides.
 *   - `stream` is a hipStream_t passed as void* (NULL = default stream).
 *   - No entry point allocates, frees or synchronizes; all work is enqueued on
 *     `stream`.  There is no mutable global state apart from the static
 *     scratch of dt_flash_fwd_ex_noalloc (see there) and write-once
 *     per-device caches (CU count, the kernels' LDS limit): calls are
 *     thread-safe.
 *   - Return value: DT_OK (0) or a negative dt_status; dt_last_error() gives
 *     a message for the calling thread's last failure.
 *   - Runtime lengths: the entry points that take a key length (kv_len) or
 *     a valid length also take it in device memory (`kv_len_dev`,
 *     `valid_len_dev`: int32, or NULL).  The kernels then read it when
 *     they run, so one captured HIP graph serves every length, as the
 *     reference's traced kv_len scalar lets one compiled program do
 *     (kernels/splash.py:583-620, models/minimax_h3/jax_server.py:271-289).
 *     The launch is then planned for every row (Skv / S), and the host
 *     length argument is the number of int32 entries the pointer holds:
 *     0 or 1 (one length for every batch element) or B (entry b for batch
 *     element b: the per-sample lengths of a CFG pair whose prompts differ,
 *     models/moss_image/jax_dit.py:181-210); any other count is DT_ERR_ARG.
 *     A device value <= 0 means no keys (attention writes zeros, and
 *     residual o = m = l = 0; the V pack and key smoothing write zero rows;
 *     the prologue zeroes every row of that batch element); a value above
 *     Skv / S is clamped to it.  Host lengths are range checked instead.
 *   - Version 0.3.0 (dt_version() == 300) changed the meaning of the host
 *     length beside a device length (above) and of a device length <= 0.
 *     Version 0.2.1 had changed six signatures (dt_qk_norm_rope,
 *     dt_qk_norm_rope_table, dt_pack_v, dt_flash_fwd_ex, dt_smooth_keys,
 *     dt_fixed_m_prepare: a device-length pointer after the host length);
 *     callers built against 0.2.0 must be rebuilt.
 */
#ifndef DT_ATTENTION_H_
#define DT_ATTENTION_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum dt_status {
  DT_OK = 0,
  DT_ERR_ARG = -1,         /* null pointer, bad enum, bad scalar */
  DT_ERR_SHAPE = -2,       /* inconsistent or non-positive sizes */
  DT_ERR_UNSUPPORTED = -3, /* head dim / alignment the kernels do not cover */
  DT_ERR_LAUNCH = -4       /* the HIP runtime rejected the launch */
};

/* RoPE channel convention (see dt_qk_norm_rope). */
enum dt_rope_mode {
  DT_ROPE_NONE = 0, /* RMSNorm only */
  DT_ROPE_HALF = 1, /* rotate-half: pair j = channels (j, j + rotary/2);
                       models/minimax_h3/jax_dit.py:251-262,
                       models/moss_image/jax_dit.py:136-142 */
  DT_ROPE_PAIR = 2  /* interleaved complex pairs (2j, 2j+1);
                       models/qwen_image_21/jax_dit.py:214-220 */
};

/* Block-sparse table granularity (dt_flash_fwd_blocksparse). */
#define DT_SPARSE_Q_BLOCK 256 /* query rows per table row */
#define DT_SPARSE_KV_TILE 64  /* keys per listed tile */

/* Library version (major*10000 + minor*100 + patch). */
int dt_version(void);

/* Message for the calling thread's most recent failed call ("" if none). */
const char* dt_last_error(void);

/*
 * Fused QK-RMSNorm + RoPE.
 *
 * For every batch b < B, token s < S and head h < H, and for q (weights wq)
 * and k (weights wk) alike:
 *     y = x * rsqrt(mean_D(x^2) + eps) * w            (fp32)
 *     y = rope(y, pos[s], axis_dims, theta, mode)       (fp32)
 *     y = y * q_head_scale[h]                           (q only, if non-NULL)
 *     out = bf16(y), or 0 when s >= valid_len
 * RMSNorm follows models/minimax_h3/jax_dit.py:191-195.  The leading
 * rotary = axis_dims[0]+axis_dims[1]+axis_dims[2] channels rotate, the rest
 * pass through (jax_dit.py:251-262); rotation pair j belongs to axis a
 * (axes own axis_dims[a]/2 consecutive pairs), has frequency
 * theta^(-2i/axis_dims[a]) for its index i inside the axis and angle
 * pos[s*3 + a] * frequency (jax_dit.py:603-617 with axis_dims = 32,32,32;
 * qwen_image_21 axes_dims_rope 16,56,56 with DT_ROPE_PAIR).
 *
 * q, k          : inputs, element (b,s,h,d) at b*in_strides[0] +
 *                 s*in_strides[1] + h*in_strides[2] + d (same for q and k).
 * q_out, k_out  : outputs, same indexing with out_strides.  May alias the
 *                 inputs only when the strides are equal (in-place).
 * wq, wk        : fp32 [D] RMSNorm weights.
 * q_head_scale  : fp32 [H] factor applied to q only, or NULL.
 * pos           : int32 [S][3] positions (t, h, w); may be NULL when
 *                 mode == DT_ROPE_NONE.
 * axis_dims     : int32 [3] channel counts per axis, even, sum <= D; with
 *                 DT_ROPE_HALF, sum/2 must be a multiple of 8.
 * valid_len     : rows s >= valid_len are written as zeros (-1: none).
 * valid_len_dev : the same in device memory (int32, one for the batch or
 *                 B of them; valid_len is then their count), or NULL; see
 *                 "Runtime lengths" (<= 0: every row zeroed, > S: none).
 * Supported D: 64, 128.  Strides must be multiples of 8 elements and the
 * pointers 16-byte aligned.
 */
int dt_qk_norm_rope(const uint16_t* q, const uint16_t* k, uint16_t* q_out,
                    uint16_t* k_out, int B, int S, int H, int D,
                    const int64_t* in_strides, const int64_t* out_strides,
                    const float* wq, const float* wk, float eps,
                    const float* q_head_scale, int mode, const int32_t* pos,
                    const int32_t* axis_dims, float theta, int valid_len,
                    const int32_t* valid_len_dev, void* stream);

/*
 * dt_qk_norm_rope with fp32 q and k (the same arguments and results; the
 * outputs are bf16).  For callers whose projections produce fp32, such as
 * the fp32 plumbing configuration: it reads the fp32 rows directly instead
 * of a separate cast to bf16 first, which also keeps the RMSNorm input
 * unrounded as the reference computes it (models/minimax_h3/jax_dit.py:
 * 191-195 takes its input dtype).  Strides in fp32 elements, multiples of 8.
 */
int dt_qk_norm_rope_f32(const float* q, const float* k, uint16_t* q_out,
                        uint16_t* k_out, int B, int S, int H, int D,
                        const int64_t* in_strides, const int64_t* out_strides,
                        const float* wq, const float* wk, float eps,
                        const float* q_head_scale, int mode,
                        const int32_t* pos, const int32_t* axis_dims,
                        float theta, int valid_len,
                        const int32_t* valid_len_dev, void* stream);

/*
 * dt_qk_norm_rope with a table-driven rotation.  Replaces the same stage as
 * dt_qk_norm_rope when the model supplies cos/sin tables instead of
 * positions: H3's apply_rope with (cos, sin) of width rotary
 * (models/minimax_h3/jax_dit.py:251-262, the torch processor's rotary_emb)
 * and MOSS's _rotate over [sin | cos] rows (models/moss_image/jax_dit.py:
 * 136-142).
 *
 * Rotation pair j < rot/2 (channels (j, j + rot/2) for DT_ROPE_HALF,
 * (2j, 2j + 1) for DT_ROPE_PAIR) of token (b, s) turns by the angle whose
 * cosine is cos_tab[b*tab_strides[0] + s*tab_strides[1] + j] and sine the
 * same element of sin_tab (fp32, device memory; a stride of 0 shares a
 * table across the batch).  Channels past rot pass through.  Everything
 * else as dt_qk_norm_rope; mode must be DT_ROPE_HALF or DT_ROPE_PAIR, rot
 * even, <= D, and for DT_ROPE_HALF rot/2 a multiple of 8.
 */
int dt_qk_norm_rope_table(const uint16_t* q, const uint16_t* k, uint16_t* q_out,
                          uint16_t* k_out, int B, int S, int H, int D,
                          const int64_t* in_strides,
                          const int64_t* out_strides, const float* wq,
                          const float* wk, float eps,
                          const float* q_head_scale, int mode,
                          const float* cos_tab, const float* sin_tab,
                          const int64_t* tab_strides, int rot, int valid_len,
                          const int32_t* valid_len_dev, void* stream);

/* dt_qk_norm_rope_table with fp32 q and k (as dt_qk_norm_rope_f32 is to
 * dt_qk_norm_rope): read as fp32, outputs bf16. */
int dt_qk_norm_rope_table_f32(const float* q, const float* k, uint16_t* q_out,
                              uint16_t* k_out, int B, int S, int H, int D,
                              const int64_t* in_strides,
                              const int64_t* out_strides, const float* wq,
                              const float* wk, float eps,
                              const float* q_head_scale, int mode,
                              const float* cos_tab, const float* sin_tab,
                              const int64_t* tab_strides, int rot,
                              int valid_len, const int32_t* valid_len_dev,
                              void* stream);

/*
 * Non-causal flash attention forward (kernels/splash.py:566-650).
 *
 * For every b < B, query head h < Hq, query row i < Sq:
 *     s_j  = scale * <q[b,h,i], k[b,h/(Hq/Hkv),j]>         for j < kv_len
 *     o    = sum_j softmax(s)_j v[b,h/(Hq/Hkv),j]
 * Keys j >= kv_len are masked (kernels/splash.py:216-218); kv_len <= 0
 * means Skv.  scale <= 0 means 1/sqrt(D) (kernels/splash.py:607).  Scores
 * accumulate in fp32 from bf16 q/k; softmax in fp32 with exp2; the
 * probabilities enter the PV product as bf16 (kernels/splash.py:256).
 *
 * q, k, v, o    : element (b,h,s,d) at b*X_strides[0] + h*X_strides[1] +
 *                 s*X_strides[2] + d.  o is bf16.
 * o32, m, l     : residual outputs (kernels/splash.py:665-742), all NULL for
 *                 the normalized form, all non-NULL for the residual form
 *                 (then `o` may be NULL):
 *                 o32 fp32 [B,Hq,Sq,D] unnormalized, contiguous;
 *                 m, l fp32 [B,Hq,Sq], contiguous: o32 and l are at scale
 *                 2^-m, i.e. l = sum_j exp2(scale*log2(e)*s_j - m) and
 *                 o32 = sum_j exp2(...) v_j.  m is a per-row reference with
 *                 rowmax - 13 < m <= rowmax (rowmax of scale*log2(e)*s; not
 *                 always equal to it), so shards
 *                 must be merged in LSE space (m + log2 l is exact), as the
 *                 reference requires for its fixed-m residuals.
 * mk            : fixed-m operand, fp32 [2][Hq] in device memory, or NULL
 *                 (kernels/splash.py:170-196, fixed_m_bound.py:98-118).
 *                 For head h with mk[Hq + h] > 0.5 the kernel starts
 *                 from the fixed reference m = mk[h] - 88 (in log2 units,
 *                 FIXED_M_RECENTER, fixed_m_bound.py:39-42) instead of the
 *                 first tile's maximum, and re-bases only if a sum
 *                 overflows.  mk[h] must bound every row's logits in log2
 *                 units (the Cauchy-Schwarz bound) and the gate keeps it
 *                 within the no-flush window; the residual m of such a head
 *                 is mk[h] - 88 unless a re-base raised it.  The
 *                 normalized result is the same softmax either way.
 * Supported D: 64, 128, 256 (head dim 256: a kernel of its own, one
 * wavefront per SIMD and 32-key tiles, at about 0.6 of the D = 128
 * kernel's rate; no E4M3 keys, packed V, tile table or tail split).
 * Hq % Hkv == 0.
 */
int dt_flash_fwd(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                 uint16_t* o, int B, int Hq, int Hkv, int Sq, int Skv, int D,
                 const int64_t* q_strides, const int64_t* k_strides,
                 const int64_t* v_strides, const int64_t* o_strides,
                 float scale, int kv_len, const float* mk, float* o32,
                 float* m, float* l, void* stream);

/*
 * Per-head maximum L2 row norm (kernels/fixed_m_bound.py:57-95).
 *
 *     out[h] = max(out[h], factor * max_{b < B, s < S} ||x[b,h,s,:]||_2)
 *
 * Row norms accumulate in fp32 from bf16 x.  `out` (fp32 [H], device memory)
 * is accumulated into, so it must be initialized by the caller (zeros for a
 * fresh maximum); several calls may fold into one output.  factor >= 0: 1
 * for keys (max_row_norm_per_head), scale*log2(e) for queries
 * (fixed_m_query_norms, :76-95).
 *
 * x             : element (b,h,s,d) at b*strides[0] + h*strides[1] +
 *                 s*strides[2] + d; a (B,S,H,D) tensor passes its (B,H,S)
 *                 strides in that order.
 * Supported D: 64, 128, 256.  Strides multiples of 8 elements, x 16-byte
 * aligned.
 */
int dt_max_row_norm(const uint16_t* x, int B, int H, int S, int D,
                    const int64_t* strides, float factor, float* out,
                    void* stream);

/*
 * Flash attention with E4M3 keys (qk_fp8, kernels/splash.py:420-424).
 *
 * As dt_flash_fwd, except that k8 holds E4M3 (OCP e4m3fn) key bytes, e.g.
 * from dt_quantize_e4m3, and the kernel casts q * scale * log2(e) (rounded
 * to bf16 first, as in dt_flash_fwd) to E4M3 with saturation at +-448
 * (kernels/fp8_cast.py:28-39) before the QK product, which runs on the
 * E4M3 MFMA with fp32 accumulation.  Probabilities and V stay bf16.
 * k_strides are in elements = bytes and must be multiples of 16; k8
 * 16-byte aligned.  Supported D: 128.
 */
int dt_flash_fwd_qk8(const uint16_t* q, const uint8_t* k8, const uint16_t* v,
                     uint16_t* o, int B, int Hq, int Hkv, int Sq, int Skv,
                     int D, const int64_t* q_strides, const int64_t* k_strides,
                     const int64_t* v_strides, const int64_t* o_strides,
                     float scale, int kv_len, const float* mk, float* o32,
                     float* m, float* l, void* stream);

/*
 * Saturating E4M3 cast (kernels/fp8_cast.py:28-39, E4M3_MAX = 448 from
 * kernels/e4m3.py:25):
 *
 *     y[b,h,s,d] = e4m3fn(clamp(bf16(factor * x[b,h,s,d]), -448, 448))
 *
 * rounding to nearest even.  x is bf16, y one byte per element; element
 * (b,h,s,d) at b*X_strides[0] + h*X_strides[1] + s*X_strides[2] + d.
 * Strides multiples of 8 elements; x 16-byte and y 8-byte aligned.
 * NaN inputs clamp to -448 (the reference keeps NaN).
 */
int dt_quantize_e4m3(const uint16_t* x, uint8_t* y, int B, int H, int S, int D,
                     const int64_t* x_strides, const int64_t* y_strides,
                     float factor, void* stream);

/*
 * Block-sparse flash attention (kernels/sparse_splash.py:568-662): as
 * dt_flash_fwd (k_format 0, bf16 k) or dt_flash_fwd_qk8 (k_format 1, E4M3
 * k), but query rows [256 i, 256 i + 256) of query head h attend only to the
 * keys of the 64-key tiles tile_ids[tile_span[2 (h n + i)] ..
 * tile_span[2 (h n + i) + 1]), n = ceil(Sq / 256), and below kv_len.  The
 * table is shared by every batch index.
 *
 * tile_span     : int32 [Hq][n][2] (begin, end) into tile_ids, device memory.
 * tile_ids      : int32 tile indices t (keys 64 t .. 64 t + 63), device
 *                 memory; each span lists distinct tiles with
 *                 64 t < kv_len (ascending keeps L2 reuse), and at least one,
 *                 else that block's rows come out zero (residual: o32, m, l
 *                 zero).  The reference's tables in (block_q, block_kv)
 *                 units map onto these when block_q is a multiple of 256 and
 *                 block_kv of 64 (or cover the whole sequence).
 * Supported D: 128.
 */
int dt_flash_fwd_blocksparse(const uint16_t* q, const void* k, int k_format,
                             const uint16_t* v, uint16_t* o, int B, int Hq,
                             int Hkv, int Sq, int Skv, int D,
                             const int64_t* q_strides,
                             const int64_t* k_strides,
                             const int64_t* v_strides,
                             const int64_t* o_strides, float scale, int kv_len,
                             const float* mk, const int32_t* tile_span,
                             const int32_t* tile_ids, float* o32, float* m,
                             float* l, void* stream);

/*
 * Packed V for the D = 128 kernels.  Same stage as the V operand of
 * dt_flash_fwd (kernels/splash.py:438-453 streams V tiles as (bkv, D)
 * blocks), stored so that the kernel's PV operand is one 16-byte LDS read.
 *
 * vt, per (b, kv head) slot s = b*Hkv + h: vt_tiles tiles of 64 keys,
 * tile t a contiguous [128][64] bf16 block at vt + (s*vt_tiles + t)*8192
 * whose row d holds channel d of keys 64t .. 64t+63.  Within each group of
 * 16 keys, column j holds key (j & 3) | ((j & 4) << 1) | ((j & 8) >> 1)
 * (keys 0-3, 8-11, 4-7, 12-15).  Keys from kv_end (kv_len, or Skv when
 * kv_len <= 0) to the end of the last tile are written as zeros.
 * vt_tiles: at least ceil(kv_end / 64) (ceil(Skv / 64) with kv_len_dev).
 * D must be 128.  v: [B, Hkv, Skv, 128] with element strides (b, h, s).
 * kv_len_dev: the key length in device memory (one int32, or B of them
 * with kv_len = B), or NULL ("Runtime lengths"); tiles past it are left
 * unwritten (the attention kernels do not read them).
 */
int dt_pack_v(const uint16_t* v, uint16_t* vt, int B, int Hkv, int Skv, int D,
              const int64_t* v_strides, int kv_len, const int32_t* kv_len_dev,
              int64_t vt_tiles, void* stream);

/*
 * The general attention entry point: dt_flash_fwd, dt_flash_fwd_qk8 and
 * dt_flash_fwd_blocksparse in one, with V row-major or packed and an
 * optional workspace.
 *
 * k_format 0: k bf16; 1: k E4M3 bytes (as dt_flash_fwd_qk8).  V: exactly
 * one of v (row-major, with v_strides, as dt_flash_fwd) and vt (the
 * dt_pack_v layout made with the same kv_len and vt_tiles).
 * tile_span/tile_ids: null for every key tile, else as
 * dt_flash_fwd_blocksparse.  o or (o32, m, l) as dt_flash_fwd.
 *
 * kv_len_dev: the key length in device memory (one int32, or B of them
 * with kv_len = B: one per batch element), or NULL ("Runtime lengths");
 * with it, vt must hold ceil(Skv / 64) tiles packed with the same
 * kv_len_dev, and a part of a split block that lies past the length
 * contributes nothing.  A device length <= 0 gives zero rows (residual:
 * o = m = l = 0); one above Skv is clamped to Skv.
 *
 * workspace (16-byte aligned device memory, or null): the kernels (D = 64
 * and D = 128) split the query blocks of a partly filled last round of workgroups over
 * their key tiles (2-16 parts, one workgroup each) and merge the parts'
 * (o, m, l) in LSE space, so that the last round does not leave CUs idle.
 * dt_flash_fwd_workspace_bytes(...) bytes hold the best split; a smaller
 * workspace gets the best split that fits it (fewer parts, or none).  Each
 * part rounds its probabilities to bf16 against its own reference m, so
 * results differ from the unsplit ones at bf16 rounding level.  The
 * workspace is scratch for the duration of the call on `stream`; calls that
 * share one workspace must be ordered.  null: no split.  No element of it
 * needs initializing.
 */
int dt_flash_fwd_ex(const uint16_t* q, const void* k, int k_format,
                    const uint16_t* v, const int64_t* v_strides,
                    const uint16_t* vt, int64_t vt_tiles, uint16_t* o, int B,
                    int Hq, int Hkv, int Sq, int Skv, int D,
                    const int64_t* q_strides, const int64_t* k_strides,
                    const int64_t* o_strides, float scale, int kv_len,
                    const int32_t* kv_len_dev, const float* mk,
                    const int32_t* tile_span, const int32_t* tile_ids,
                    float* o32, float* m, float* l, void* workspace,
                    size_t workspace_bytes, void* stream);

/*
 * Workspace bytes dt_flash_fwd_ex can use for this shape on the current
 * device (0: no split would help, or D is not 64 or 128; head dim 256
 * never splits).  Depends on the
 * device's compute-unit count.  Pass kv_len 0 for calls that give
 * kv_len_dev.
 */
size_t dt_flash_fwd_workspace_bytes(int B, int Hq, int Sq, int Skv,
                                    int kv_len, int D);

/*
 * The launch plan dt_flash_fwd_ex follows for this shape on the current
 * device with workspace_bytes of workspace (0: none).  plan[6] receives:
 * [0] the device's compute units, [1] the query blocks of 256 rows
 * (B * Hq * ceil(Sq / 256)), [2] the 64-key tiles per block
 * (ceil(kv_end / 64)), [3] the parts each tail block is split into (1: no
 * split), [4] the tail blocks split, [5] the blocks run whole; *ws_needed
 * the workspace bytes the plan uses.  Pass kv_len 0 for calls that give
 * kv_len_dev.  Head dim 256 plans blocks of 128 rows over 32-key tiles
 * and never splits.  This is the gfx950 side of the reference's per-shape block
 * resolution (kernels/block_sizes.py:537-577, used at
 * kernels/mesh_attention.py:198-215): the tile is fixed, and what a shape
 * decides is the tail split.
 */
int dt_flash_fwd_plan(int B, int Hq, int Sq, int Skv, int kv_len, int D,
                      size_t workspace_bytes, int32_t* plan,
                      size_t* ws_needed);

/*
 * dt_flash_fwd_ex without a workspace argument: the tail split's partial
 * (o, m, l) live in a static device array of DT_NOALLOC_SCRATCH_BYTES bytes
 * inside the library (one per GPU, held until the process ends), and the
 * call allocates nothing.  No counterpart in the reference: it is for
 * callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).
 *
 * Arguments and results as dt_flash_fwd_ex, with workspace and
 * workspace_bytes replaced by scratch_bytes: how much of the static
 * scratch the call may use, exactly as if dt_flash_fwd_ex were given a
 * workspace of that many bytes (same split, bit-identical results);
 * dt_flash_fwd_workspace_bytes(...) gives the best split's need, 0 means
 * no split.  scratch_bytes above DT_NOALLOC_SCRATCH_BYTES is rejected
 * (DT_ERR_ARG).  Nothing in the scratch needs to start at zero.  Every
 * call on one GPU shares that GPU's scratch, which keeps the last call's
 * contents: calls that overlap on one GPU (other streams, other threads)
 * race and must be ordered by the caller.
 */
#define DT_NOALLOC_SCRATCH_BYTES (64u << 20)
int dt_flash_fwd_ex_noalloc(const uint16_t* q, const void* k, int k_format,
                            const uint16_t* v, const int64_t* v_strides,
                            const uint16_t* vt, int64_t vt_tiles, uint16_t* o,
                            int B, int Hq, int Hkv, int Sq, int Skv, int D,
                            const int64_t* q_strides,
                            const int64_t* k_strides,
                            const int64_t* o_strides, float scale, int kv_len,
                            const int32_t* kv_len_dev, const float* mk,
                            const int32_t* tile_span, const int32_t* tile_ids,
                            float* o32, float* m, float* l,
                            size_t scratch_bytes, void* stream);

/*
 * Key smoothing.  Replaces the reference's
 *   mean = sum(k[:, :, :kv_len], axis=2) / kv_len   (float32)
 *   k = where(s < kv_len, k - mean.astype(bf16), 0)
 * (models/minimax_h3/jax_server.py:271-289; without kv_len the mean over all
 * rows, kernels/mesh_attention.py:234-237, backends/ours_splash_tt.py:
 * 136-137).  Softmax attention over ks equals attention over k; fixed-m's
 * bound assumes smoothed keys.
 *
 * k, ks: bf16 [B, H, S, D] with element strides (b, h, s); ks may be k
 * (in place).  kv_len <= 0: every row is real.  Row s < kv_len of ks is
 * bf16(k - m) with m the float32 mean of the real rows rounded to bf16;
 * rows s >= kv_len are zero.  norms: null, or [H] floats that receive
 * max(norms[h], max over b, s of ||ks[b, h, s, :]||) (caller zero-inits,
 * as dt_max_row_norm).  workspace: at least
 * dt_smooth_keys_workspace_bytes(B, H, S, D, kv_len) bytes, 16-byte
 * aligned, scratch for the call (sized with kv_len 0 for calls that give
 * kv_len_dev).  kv_len_dev: the length in device memory, one int32 or B of
 * them (kv_len = B: batch element b's mean is over its own rows <
 * kv_len_dev[b]), or NULL ("Runtime lengths").  Supported D: 64, 128, 256.
 * Deterministic.
 */
int dt_smooth_keys(const uint16_t* k, uint16_t* ks, int B, int H, int S, int D,
                   const int64_t* k_strides, const int64_t* ks_strides,
                   int kv_len, const int32_t* kv_len_dev, float* norms,
                   void* workspace, size_t workspace_bytes, void* stream);
size_t dt_smooth_keys_workspace_bytes(int B, int H, int S, int D, int kv_len);

/*
 * The fixed-m preparation of one attention call.  Replaces
 * kernels/fixed_m_bound.py:98-118 as kernels/splash.py:609-614 uses it:
 *   bound[h] = max_{b,s} ||q[b,h,s]|| * q_factor * max_{b,s} ||k'[b,hk,s]||
 *   mk[0][h] = ceil(bound[h]),  mk[1][h] = (bound[h] <= gate),
 * hk = h / (Hq / Hkv), q_factor = scale * log2(e), gate the no-flush gate
 * (FIXED_M_SAFE_BOUND 213 for smoothed keys).  smooth != 0: k' is k
 * smoothed as dt_smooth_keys does (mean over rows < kv_len, rows past it
 * zero) and is written to ks; smooth == 0: k' = k over all Skv rows and ks
 * is unused (may be null).  q, k, ks: bf16 [B, H, S, D] with element
 * strides (b, h, s).  mk: [2][Hq] fp32, device memory.  workspace: at least
 * dt_fixed_m_prepare_workspace_bytes(...) bytes, 16-byte aligned (sized
 * with kv_len 0 for calls that give kv_len_dev).  kv_len_dev: the length in
 * device memory, one int32 or B of them (kv_len = B), or NULL ("Runtime
 * lengths").  Supported D: 64, 128, 256.  Deterministic; mk equals the operand
 * built from
 * dt_max_row_norm (and dt_smooth_keys).
 */
int dt_fixed_m_prepare(const uint16_t* q, const uint16_t* k, uint16_t* ks,
                       int B, int Hq, int Hkv, int Sq, int Skv, int D,
                       const int64_t* q_strides, const int64_t* k_strides,
                       const int64_t* ks_strides, int kv_len,
                       const int32_t* kv_len_dev, float q_factor, float gate,
                       int smooth, float* mk, void* workspace,
                       size_t workspace_bytes, void* stream);
size_t dt_fixed_m_prepare_workspace_bytes(int B, int Hq, int Hkv, int Sq,
                                          int Skv, int D, int kv_len,
                                          int smooth);

#ifdef __cplusplus
}
#endif

#endif /* DT_ATTENTION_H_ */
