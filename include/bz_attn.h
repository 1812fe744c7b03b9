/*
 * bz_attn.h -- C ABI of the decode-step attention in libbzgemv.so (gfx950):
 * the step between the QKV and o_proj GEMVs of a fused decoder layer, one
 * new token per batch row against a static KV cache.
 *
 * Conventions are those of bz_gemv.h (device pointers owned by the caller,
 * stream = hipStream_t as void*, errors detected on the host before any
 * launch, no allocation or host synchronization, bf16 = raw uint16).
 *
 * Shapes: B batch rows, HQ query heads, HKV key/value heads (HQ % HKV == 0),
 * head dim D, static cache length S.
 *   qkv      bf16 [B][ld_qkv], columns [q heads | k heads | v heads] x D
 *   cos/sin  [B][D] with batch stride ld_cs, or one row with ld_cs = 0;
 *            bf16 or fp32 (cs_dtype)
 *   caches   [B][HKV][S][D], bf16 or fp32 (cache_dtype)
 *   pos      device int64 scalar: the cache position of the new token.  A
 *            position outside [0, S) writes no cache entry; attention covers
 *            positions [0, min(pos, S - 1)], none for pos < 0 (output 0).
 *   mask     [B][ld_mask], column s = cache position s; ld_mask = 0 gives
 *            every row the same mask.  mask_dtype BZ_DT_BF16 / BZ_DT_F32:
 *            additive; BZ_MASK_BOOL: uint8, nonzero = attend (adds 0), zero
 *            adds -1e30 (the conversion of _additive_mask,
 *            models/fused/kernels.py:492-502, done per read, so a mask
 *            buffer updated in place is never stale)
 *   q_out    fp32 [B][HQ][D]
 *   out      bf16 [B][ld_out], query head h at columns h*D .. h*D+D-1
 */
#ifndef BZ_ATTN_H
#define BZ_ATTN_H

#include <stddef.h>
#include <stdint.h>

#include "bz_gemv.h"

#ifdef __cplusplus
extern "C" {
#endif

#define BZ_ATTN_MAX_SPLIT 64
#define BZ_MASK_BOOL 2

/* Per-head q/k RMSNorm (q_norm/k_norm bf16 [D], both or neither), rotate-half
 * RoPE with cos/sin, q to q_out, new k (normed, rotated) and v written into
 * the caches at pos.  Replaces qkv_rope_cache_kernel with _rms_head and
 * _rope, models/fused/kernels.py:356-401 (launched from attention_step,
 * :521-526).  D even, D <= 1024.
 * seq_len (nullable, device int64) is set to pos + 1: the fill counter of a
 * cache whose own update writes at its counter rather than at pos
 * (transformers >= 5 StaticLayer.cumulative_length), kept in step so fused
 * and unfused calls on one cache agree.  No counterpart in the reference,
 * whose transformers (4.57) cache writes at cache_position. */
int bz_qkv_rope_cache(const void* qkv, int64_t ld_qkv, int32_t B, int32_t HQ,
                      int32_t HKV, int32_t D, const void* q_norm,
                      const void* k_norm, float eps, const void* cos,
                      const void* sin, int32_t cs_dtype, int64_t ld_cs,
                      const int64_t* pos, float* q_out, void* k_cache,
                      void* v_cache, int32_t S, int32_t cache_dtype,
                      int64_t* seq_len, void* stream);

/* out = softmax(q k^T * scale + mask) v over cache positions [0, pos], per
 * query head, with query head h reading kv head h / (HQ / HKV); q fp32
 * [B][HQ][D] already normed and rotated.  One launch: a workgroup per
 * (batch row, kv head, split) with the positions cut into `split` equal
 * ranges; for split > 1 the last workgroup of each (row, kv head) to finish
 * combines the ranges, through `workspace` (bz_attn_workspace bytes, zeroed
 * once before its first use: the kernel leaves its arrival counters at zero
 * again).  While at most 160 positions are attended (decided on the device
 * from *pos) the call runs unsplit whatever `split` says: the workgroup of
 * split 0 covers every position and writes the output, the others return at
 * once and the workspace is not touched.  Calls that share a workspace must
 * not overlap.  Replaces
 * attn_decode_kernel + attn_combine_kernel, models/fused/kernels.py:404-475
 * (attention_step :528-536 picks split 1 for S <= 256, else 8;
 * bz_attn_default_split is this build's choice).
 * D in {64, 128, 256, 512}; HQ / HKV <= 16 (<= 4 for D = 512). */
int bz_attn_decode(const float* q, const void* k_cache, const void* v_cache,
                   int32_t cache_dtype, int32_t B, int32_t HQ, int32_t HKV,
                   int32_t D, int32_t S, const void* mask,
                   int32_t mask_dtype, int64_t ld_mask,
                   const int64_t* pos, float scale, int32_t split,
                   void* workspace, void* out, int64_t ld_out, void* stream);

/* The whole attention step of a decode token in one launch: the work of
 * bz_qkv_rope_cache (q/k RMSNorm, RoPE, new k and v into the caches at pos,
 * seq_len = pos + 1 when given; seq_len must not alias pos) and of
 * bz_attn_decode, with q never leaving the chip and the new token's k and v
 * taken from the workgroup's own registers.  Replaces attention_step,
 * models/fused/kernels.py:505-536 (three launches there).  Same limits and
 * workspace as bz_attn_decode. */
int bz_attn_step(const void* qkv, int64_t ld_qkv, int32_t B, int32_t HQ,
                 int32_t HKV, int32_t D, const void* q_norm,
                 const void* k_norm, float eps, const void* cos,
                 const void* sin, int32_t cs_dtype, int64_t ld_cs,
                 const int64_t* pos, void* k_cache, void* v_cache, int32_t S,
                 int32_t cache_dtype, int64_t* seq_len, const void* mask,
                 int32_t mask_dtype, int64_t ld_mask, float scale,
                 int32_t split, void* workspace, void* out, int64_t ld_out,
                 void* stream);

/* Workspace bytes of bz_attn_decode / bz_attn_step (0 for split == 1): the
 * fp32 split partials [B][HQ][split][D + 4] and B * HKV arrival counters.
 * Replaces the partial-buffer cache _attn_partials,
 * models/fused/kernels.py:481-489. */
size_t bz_attn_workspace(int32_t B, int32_t HQ, int32_t HKV, int32_t D,
                         int32_t split);

/* Split count for a static cache of S positions: about 128 positions per
 * workgroup at a full cache, between 1 and 32. */
int32_t bz_attn_default_split(int32_t S);

#ifdef __cplusplus
}
#endif

#endif /* BZ_ATTN_H */
