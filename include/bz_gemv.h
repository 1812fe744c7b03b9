/*
 * bz_gemv.h -- C ABI of libbzgemv.so, the MI355X (gfx950) decode-time linear
 * layers of Breeze TTS 2: RMSNorm-prologue GEMV over int4 group-quantized,
 * fp8 e4m3 (OCP) per-row-scaled or bf16 weights, with a SiLU-gate or residual
 * epilogue, plus the load-time quantizers and two small glue kernels.
 *
 * Conventions
 *   - Every pointer argument is a device pointer owned by the caller, except
 *     the descriptor itself (host memory, read during the call only).
 *   - `stream` is a hipStream_t passed as void* (NULL = the null stream).
 *   - No call allocates memory, synchronizes the host or tunes anything, so
 *     every call can be recorded into a HIP graph.  Calls on different
 *     streams are independent as long as they do not share a workspace (the
 *     caller's; bz_gemv_noalloc is the one exception: its static array is one
 *     per GPU, shared by every stream, see there).
 *   - Return value: BZ_OK (0) or a bz_status error code; bz_strerror() names
 *     it.  Invalid descriptors and arguments are rejected on the host before
 *     anything is launched.
 *   - bfloat16 tensors are raw uint16 bit patterns; "bf16" below.
 */
#ifndef BZ_GEMV_H
#define BZ_GEMV_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define BZ_ABI_VERSION 4

typedef enum bz_status {
    BZ_OK = 0,
    BZ_ERR_INVALID_ARG = 1,  /* null pointer, bad enum, non-positive size  */
    BZ_ERR_SHAPE = 2,        /* K not divisible by the group / format step */
    BZ_ERR_ALIGNMENT = 3,    /* pointer or leading dimension misaligned    */
    BZ_ERR_UNSUPPORTED = 4,  /* a valid request this build cannot run      */
    BZ_ERR_LAUNCH = 5,       /* the HIP runtime rejected a launch          */
    BZ_ERR_ABI = 6,          /* descriptor abi_version mismatch            */
    BZ_ERR_SCRATCH = 7       /* bz_gemv_noalloc: the call needs more workspace
                                than BZ_GEMV_SCRATCH_BYTES                  */
} bz_status;

/* Weight formats.  All weights are row-major over the N output channels.
 *
 * BZ_W_INT4_ZP : w uint8 [N][K/2]; byte j of row n holds k = 2j in the low
 *                nibble and k = 2j+1 in the high nibble (q in 0..15).
 *                sc0 = scales_zeros bf16 [K/group][N][2] = (s, z);
 *                w_eff = (q - 8) * s + z.   This is the byte layout of the
 *                rebuilt Int4Linear.weight_int4 and the exact scales_zeros of
 *                models/int4_linear.py:61-63.
 * BZ_W_INT4_MIN: same nibbles; sc0 = scale bf16 [N][K/group], sc1 = min bf16
 *                [N][K/group]; w_eff = q * s + min
 *                (models/fused/kernels.py:141-150, FusedWeight bits=4).
 * BZ_W_FP8     : w uint8 [N][K] OCP e4m3 ("e4m3fn") codes; sc0 = float
 *                [N] per-output-channel scale, applied to the fp32 dot
 *                product (models/fused/kernels.py:124-126,133-134;
 *                Fp8Linear.weight_fp8 / weight_scale, models/fp8_linear.py:62-66).
 * BZ_W_BF16    : w bf16 [N][K]; sc0/sc1 unused (FusedWeight bits=16).
 *
 * Tiled formats (the layout the streaming GEMV path reads fastest; written by
 * bz_pack_tiled, bz_tiled_bytes bytes, N % 16 == 0):
 *   A row block is 16 weight rows; a unit is 64 bytes of each row (int4: 128
 *   k = one group of 128; fp8: 64 k).  Row block b occupies one contiguous
 *   chunk: its K/unit tiles of 1024 bytes (tile u = unit u of the 16 rows, row
 *   r at byte 64 r, bytes in row-major order), then its scales, padded to a
 *   multiple of 128 bytes:
 *     int4: per unit u and row r the (s, z) bf16 pair at byte 64 u + 4 r,
 *           w_eff = (q - 8) * s + z  (the BZ_W_INT4_ZP semantics, group 128);
 *     fp8:  the 16 fp32 row scales.
 *   sc0 / sc1 are unused (the scales travel in w).
 * BZ_W_INT4_TILED / BZ_W_FP8_TILED: block b holds rows 16b .. 16b+15.
 * BZ_W_*_TILED_PAIRED: the [gate; up] weight of a SiLU-gate GEMV
 *   (models/fused/layer.py:60; N = 2 * N_out): block b holds gate rows
 *   8b .. 8b+7 then up rows 8b .. 8b+7 (logical rows 8b+r and N/2+8b+r), so a
 *   block finishes 8 outputs silu(g) * u.  Only valid with BZ_EPI_SILU_GATE;
 *   the unpaired tiled formats do not take that epilogue.
 * The tiled formats run on GEMV path 5, the streaming kernel (M <= 8 rows
 * per launch; more rows run as several launches), and the unpaired ones also
 * on the several-row paths 4 and 6 (see below).  They need K % 128 == 0
 * (int4) or K % 64 == 0 (fp8); int4 group must be 128.
 */
typedef enum bz_wfmt {
    BZ_W_INT4_ZP = 0,
    BZ_W_INT4_MIN = 1,
    BZ_W_FP8 = 2,
    BZ_W_BF16 = 3,
    BZ_W_INT4_TILED = 4,
    BZ_W_INT4_TILED_PAIRED = 5,
    BZ_W_FP8_TILED = 6,
    BZ_W_FP8_TILED_PAIRED = 7
} bz_wfmt;

/* Epilogues of models/fused/kernels.py:8-13 (EPI 0/1/2). */
typedef enum bz_epilogue {
    BZ_EPI_NONE = 0,
    BZ_EPI_SILU_GATE = 1,  /* out[m,j] = silu(acc[m,j]) * acc[m,j+N/2]; N_out = N/2 */
    BZ_EPI_RESIDUAL = 2    /* out[m,n] = acc[m,n] + residual[m,n]                   */
} bz_epilogue;

typedef enum bz_dtype {
    BZ_DT_BF16 = 0,
    BZ_DT_F32 = 1
} bz_dtype;

/* One GEMV call: out[M, N_out] = epilogue( rmsnorm(x) @ w_eff^T ).
 *
 * x is bf16 [M][ldx] (ldx >= K, x and every row 16-byte aligned: ldx % 8 == 0).
 * gamma (bf16 [K]) != NULL enables the fused RMSNorm
 *   out = rsqrt(mean(x^2) + eps) * (bf16(x * gamma) @ w_eff^T)   (fp32 math),
 * i.e. rmsnorm(x) @ w_eff^T with the per-row scalar applied after the dot
 * product, computed inside the kernel from the full row of x
 * (models/fused/kernels.py:65-81).  Accumulation is fp32.
 * residual (dtype residual_dtype, [M][ldr]) is read only for BZ_EPI_RESIDUAL
 * and may alias `out`.  out is [M][ldo] of out_dtype.
 * cfg_depth / cfg_waves / cfg_tiles / cfg_path: 0 selects the built-in
 * per-shape rule; otherwise they force the streaming kernel's pipeline depth
 * (2, 4, 8 or 16 steps of weight loads in flight per wave; at most 8 for
 * SiLU-gate), waves per workgroup (1..8), output tiles per workgroup (>= 1)
 * and arithmetic path (1 = v_dot2 kernel, 8-column tiles; 2 = bf16 MFMA
 * kernel, 16-column tiles, needs an int4 group >= 128; 3 = int8 MFMA kernel
 * for int4 weights, group >= 128 and K % 128 == 0, x held as two int8
 * planes per row (about 16 significant bits), up to 16 rows per launch;
 * 4 = several-row bf16 MFMA tile kernel, see below; 5 = the streaming
 * kernels of the tiled formats: cfg_tiles = 0 the one-block kernel (one
 * 16-row block per workgroup), cfg_tiles = 1..8 the several-block kernel
 * with that many consecutive row blocks per workgroup, cfg_waves 1..16
 * waves per workgroup (0 = the kernel's rule), cfg_depth unused; 6 = the
 * several-row panel kernel of the tiled formats, see below).  Without a cfg
 * the rule takes the several-block kernel for weights of more than 256 row
 * blocks (one workgroup per CU), for fp8 rows of 64 units or more, and for
 * 3-8 rows of an unpaired weight without RMSNorm over K <= 8192 (one block
 * per workgroup, all rows in one launch).  Used by tuning sweeps.
 *
 * Several rows (path 4).  Up to 32 rows of x per launch stream every weight
 * byte once: a workgroup of cfg_waves waves (4 or 8) owns 16 * cfg_tiles
 * output columns per wave (cfg_tiles 1 or 2) and one of cfg_slices K slices
 * (0: the built-in rule, x slice <= 80 KB of LDS).  It needs no
 * RMSNorm (gamma NULL), epilogue NONE or RESIDUAL, an int4 group >= 128 and
 * K a multiple of 128 (int4), 64 (fp8) or 32 (bf16); larger M runs 32 rows
 * per launch.  With more than one K slice the slices' fp32 partials go to
 * `workspace` (bz_gemv_workspace bytes, 16-byte aligned, zero-filled before
 * its first use; every call leaves its counters zero again, so it is never
 * cleared afterwards and calls can be recorded into a graph).  Calls that
 * share a workspace must not run concurrently.  The automatic rule takes
 * this path from M = 5 on when `workspace` is large enough (or none is
 * needed), else it keeps the row-sliced paths.
 *
 * Several rows over the tiled formats (path 6, the panel kernel).  Up to 32
 * rows of x per launch against an unpaired tiled int4 or fp8 weight
 * (BZ_W_INT4_TILED, BZ_W_FP8_TILED), no RMSNorm, epilogue NONE or RESIDUAL,
 * no second store: each workgroup of cfg_waves waves (0: about 5 units per
 * wave; at most 16, or 8 with several blocks) covers cfg_tiles consecutive
 * 16-row blocks (1..5; 0: enough to keep about 256 workgroups, or with K
 * slices 2 (int4) / 3 (fp8), one per 48 blocks for fewer) over the whole K
 * or over one of cfg_slices K slices (0: one, or, for K >= 8192 with more
 * than 128 KB of x per launch or N < 2048, about 240 workgroups in all
 * where that makes at least two slices); larger M runs 32 rows per launch.  With more than
 * one slice the slices' fp32 sums go to `workspace` as for path 4
 * (bz_gemv_workspace bytes); forced slices without it return
 * BZ_ERR_INVALID_ARG, and the rule's slices without it fall back to the
 * whole K.  The automatic rule takes this path for these weights from M = 5
 * on, except 5-8 rows over K <= 8192 that the several-block streaming
 * kernel runs in one launch; the streaming kernels otherwise.
 */
typedef struct bz_gemv_desc {
    int32_t abi_version;      /* must be BZ_ABI_VERSION */
    int32_t M, N, K;          /* N = weight rows (2*N_out for SiLU-gate) */
    int32_t group;            /* int4 group size (power of two >= 32) */
    int32_t wfmt;             /* bz_wfmt */
    int32_t epilogue;         /* bz_epilogue */
    int32_t out_dtype;        /* bz_dtype */
    int32_t residual_dtype;   /* bz_dtype */
    int32_t cfg_depth, cfg_waves, cfg_tiles, cfg_path;  /* 0 = automatic */
    int32_t cfg_slices;       /* paths 4 and 6: K slices (0 = automatic) */
    float eps;
    const void* x;  int64_t ldx;
    const void* w;
    const void* sc0;
    const void* sc1;
    const void* gamma;
    const void* residual; int64_t ldr;
    void* out; int64_t ldo;
    void* workspace; size_t workspace_bytes;  /* path 4 split-K partials + counters */
    /* Second store (tiled formats only): output columns [0, n_out2) are also
     * written to out2 (same dtype as out, leading dimension ldo2), e.g. the
     * query part of a QKV projection into the buffer of the next kernel.
     * n_out2 = 0 disables it. */
    void* out2; int64_t ldo2;
    int32_t n_out2; int32_t reserved0;  /* reserved0 must be 0 */
} bz_gemv_desc;

/* ABI version of the loaded library (BZ_ABI_VERSION it was built with). */
int bz_abi_version(void);

/* Static description of a status code. */
const char* bz_strerror(int status);

/* Host helper, no counterpart in the reference: *active = 1 and *id = the
 * capture's id while a graph capture is under way on `stream`, else 0 and 0.
 * Launches nothing.  The torch binding keys its GEMV and attention
 * workspaces by (device, stream) and, during a capture, by the capture, so
 * calls on different streams and different captured graphs never share one
 * (the reference's one cached partial buffer per device,
 * models/fused/kernels.py:179,192-198, is shared by every stream). */
int bz_stream_capture(void* stream, int32_t* active, uint64_t* id);

/* Workspace bytes the several-row kernels (the tile path 4, the panel path
 * 6) need for this descriptor: 0 when bz_gemv would take neither (M < 5
 * without cfg_path 4 or 6, an RMSNorm or SiLU-gate call, unsupported K or
 * group) or runs it with a single K slice.  Returns 0 for an invalid
 * descriptor. */
size_t bz_gemv_workspace(const bz_gemv_desc* d);

/* The fused decode GEMV.  Replaces, as one launch:
 *   rms_gemv + _launch (rms_gemv_kernel + gemv_epilogue_kernel)
 *       models/fused/kernels.py:201-219, 334-351
 *   torch._weight_int4pack_mm in Int4Linear.forward
 *       models/int4_linear.py:103-108
 *   torch._scaled_mm in Fp8Linear.forward (weight-only form, bf16
 *       activations) models/fp8_linear.py:76-82
 * Any M >= 1 is accepted (the reference fused kernel stops at M <= 2,
 * models/fused/kernels.py:336). */
int bz_gemv(const bz_gemv_desc* d, void* stream);

/* Measurement aid, no counterpart in the reference: reads `bytes` (a
 * multiple of `chunk`, which is a multiple of 16 and at most 256 KiB;
 * 16-byte aligned) from device memory `p` once, one workgroup per
 * contiguous `chunk` bytes (1 KiB tiles, about 4 per wave), and
 * writes nothing unless the XOR a thread read equals `key` (then `*sink`).
 * Its duration is the streaming-read floor the GEMVs are compared with, for
 * the same bytes per workgroup; bytes = 0 launches one empty workgroup (the
 * fixed cost of a launch). */
int bz_stream_read(const void* p, size_t bytes, size_t chunk, uint32_t key, uint32_t* sink, void* stream);

/* Measurement aid, no counterpart in the reference: `workgroups` workgroups
 * of 1024 threads each read all `xbytes` of `x` (the same bytes for every
 * workgroup; at most 64 MiB) and their own `wchunk` bytes of `w` (workgroup
 * b at w + b * wchunk; at most 16 MiB), 16-byte aligned sizes and pointers,
 * and write nothing unless a thread's XOR equals `key`.  Its duration is the
 * floor of a several-row GEMV whose workgroups each cover the whole K (every
 * one streams all of x from L2 beside its weights). */
int bz_shared_read(const void* x, size_t xbytes, const void* w, size_t wchunk, int workgroups, uint32_t key,
                   uint32_t* sink, void* stream);

/* Size of bz_gemv_noalloc's static device workspace, per GPU. */
#define BZ_GEMV_SCRATCH_BYTES ((size_t)8 << 20)

/* bz_gemv without allocation: identical results and kernels, with the
 * descriptor's workspace fields ignored and replaced by a static device
 * array of BZ_GEMV_SCRATCH_BYTES that the library holds per GPU until the
 * process ends.  No counterpart in the reference: it is for callers that
 * cannot allocate device memory (code under graph capture, serving loops and
 * harnesses that forbid hipMalloc), which otherwise would have to pass a
 * workspace.  Allocates nothing (no hipMalloc, no library allocation).
 * Returns BZ_ERR_SCRATCH when bz_gemv_workspace(d) exceeds
 * BZ_GEMV_SCRATCH_BYTES, else what bz_gemv returns.  The first call on a
 * device looks up that device's copy of the array and clears its counters
 * on `stream`.  All calls on one GPU share its array: calls that overlap in
 * time on one GPU (concurrent streams, host threads) race and must not be
 * made. */
int bz_gemv_noalloc(const bz_gemv_desc* d, void* stream);

/* Row RMSNorm, out = bf16(x * rsqrt(mean(x^2)+eps) * gamma); bf16 in/out.
 * Replaces rmsnorm / rmsnorm_kernel, models/fused/kernels.py:541-557. */
int bz_rmsnorm(const void* x, int64_t ldx, const void* gamma, float eps,
               void* out, int64_t ldo, int32_t M, int32_t K, void* stream);

/* out = silu(g) * u, bf16 in/out.
 * Replaces silu_mul / silu_mul_kernel, models/fused/kernels.py:560-575. */
int bz_silu_mul(const void* g, int64_t ldg, const void* u, int64_t ldu,
                void* out, int64_t ldo, int32_t M, int32_t N, void* stream);

/* Group int4 quantizer (load time).  w is [N][K] float32 (w_dtype BZ_DT_F32)
 * or bf16 (BZ_DT_BF16).  symmetric = 0: min/max quantizer of
 * quantize_int4 (models/int4_linear.py:47-63) and pack_int4
 * (models/fused/kernels.py:141-150); symmetric = 1: s = absmax/7,
 * q = clamp(rne(w/s)+8, 0, 15), z = 0.
 * Writes packed uint8 [N][K/2] (even-k low nibble) and, for
 * layout BZ_W_INT4_ZP, sc0 = scales_zeros bf16 [K/group][N][2];
 * for BZ_W_INT4_MIN, sc0 = scale bf16 [N][K/group], sc1 = min bf16.
 * Replaces quantize_int4 + torch._convert_weight_to_int4pack
 * (models/int4_linear.py:47-64) and pack_int4. */
int bz_quantize_int4(const void* w, int32_t w_dtype, int32_t N, int32_t K,
                     int32_t group, int32_t symmetric, int32_t layout,
                     void* packed, void* sc0, void* sc1, void* stream);

/* Per-output-channel fp8 e4m3 quantizer (load time): scale = max(amax,
 * amax_floor)/448, code = e4m3(clamp(w/scale, -448, 448)) with round to
 * nearest even.  amax_floor = 1e-12 is Fp8Linear.__init__
 * (models/fp8_linear.py:58-62); 1e-8 is pack_fp8
 * (models/fused/kernels.py:153-158).  Writes codes uint8 [N][K] and
 * scale float [N]. */
int bz_quantize_fp8(const void* w, int32_t w_dtype, int32_t N, int32_t K,
                    float amax_floor, void* codes, void* scale, void* stream);

/* Bytes of a tiled weight (wfmt one of the BZ_W_*_TILED formats) of N rows
 * and K columns; 0 when the shape cannot be tiled (N % 16, or K not a
 * multiple of the unit's 128 (int4) / 64 (fp8) values). */
size_t bz_tiled_bytes(int32_t wfmt, int32_t N, int32_t K);

/* Write logical rows [row0, row0 + n) of a tiled weight of N rows (dst,
 * bz_tiled_bytes(dst_wfmt, N, K) bytes, 16-byte aligned) from a source of n
 * rows: row-major BZ_W_INT4_ZP (group 128; src_sc0 = scales_zeros bf16
 * [K/128][n][2]) or BZ_W_INT4_TILED (n % 16 == 0, src_sc0 unused) for the
 * int4 tiled formats; BZ_W_FP8 (src_sc0 = float [n] row scales) or
 * BZ_W_FP8_TILED for the fp8 ones.  For the paired formats logical row r < N/2 is
 * gate row r and r >= N/2 up row r - N/2, so [gate; up] is packed by one call
 * over all N rows or by one call per half (row0 = 0, row0 = N/2).  Load-time
 * work with no counterpart in the reference: it replaces the repack step of
 * torch._convert_weight_to_int4pack (models/int4_linear.py:59) by this
 * build's own layout.  Bytes a call does not cover (chunk padding, rows of
 * other calls) are left as they are. */
int bz_pack_tiled(int32_t src_wfmt, const void* src_w, const void* src_sc0, int32_t n, int32_t K, int32_t group,
                  int32_t dst_wfmt, void* dst, int32_t N, int32_t row0, void* stream);

/* Dequantize any weight format to float [N][K] (w_eff of bench_gemv.py:47-52)
 * with the same device unpacking code as bz_gemv.  Used to pin unpacking and
 * indexing bit-exactly, and for checkpoint export.  Tiled formats write the
 * logical row order (for the paired ones [gate; up]); group must be 128 for
 * the int4 tiled formats and sc0/sc1 are ignored. */
int bz_dequant(int32_t wfmt, const void* w, const void* sc0, const void* sc1,
               int32_t N, int32_t K, int32_t group, void* out, void* stream);

/* fp32 head GEMV: out[m][n] = sum_k x[m][k] * W[n][k], x, W and out fp32
 * (fp32 products and sums).  W is one of nmat matrices [N][K] (K contiguous,
 * 16-byte aligned rows) mat_stride floats apart, chosen on the device:
 * sel = (index ? *index : 0) + index_offset, W = w + sel * mat_stride; a
 * selection outside [0, nmat) writes zeros.  K % 4 == 0, K <= 4096.
 * Replaces the fp32 head matmuls the reference keeps unquantized:
 *   lm_head cast to fp32, input cast to fp32
 *       models/cudagraph/backbone_graph.py:69-70,273
 *   BreezeCodebooksHead.forward, codebook cache_position - 1
 *       models/breeze.py:597-612, models/cudagraph/depth_decoder_graph.py:159-161
 *       (its [hidden][vocab] weight is used here transposed to [vocab][hidden]) */
int bz_head_f32(const float* x, int64_t ldx, int32_t M, int32_t K,
                const float* w, int32_t N, int64_t mat_stride, int32_t nmat,
                const int64_t* index, int64_t index_offset, float* out,
                int64_t ldo, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* BZ_GEMV_H */
