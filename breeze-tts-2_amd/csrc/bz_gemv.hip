// Host dispatcher of the streaming decode GEMV (C ABI entry bz_gemv).  The
// kernels are in bz_gemv_kernel.h (dot2 path), bz_gemv_mfma.h (bf16
// matrix-core path), bz_gemv_i8.h (int8 matrix-core path for int4 weights),
// bz_gemv_tile.h (several-row tile kernel), bz_gemv_stream.h (the tiled
// formats' streaming kernel) and bz_gemv_panel.h (their several-row
// kernel); their instances live in
// bz_gemv_{,mfma_,i8_,tile_,stream_,panel_}<fmt>.hip.
#include <algorithm>

#include "bz_gemv_panel.h"
#include "bz_gemv_tile.h"
#include "bz_gemv_wide.h"

namespace bz {

enum { PATH_DOT2 = 1, PATH_MFMA = 2, PATH_I8 = 3, PATH_TILE = 4, PATH_STREAM = 5, PATH_PANEL = 6 };

static int launch_wf(int wf, int path, const GemvParams& p, const Launch& l, hipStream_t st) {
    if (path == PATH_I8) {
        if (wf == WF_I4ZP) return launch_i8_i4zp(p, l, st);
        if (wf == WF_I4MIN) return launch_i8_i4min(p, l, st);
        return BZ_ERR_INVALID_ARG;
    }
    const bool mfma = path == PATH_MFMA;
    switch (wf) {
        case WF_I4ZP: return mfma ? launch_mfma_i4zp(p, l, st) : launch_i4zp(p, l, st);
        case WF_I4MIN: return mfma ? launch_mfma_i4min(p, l, st) : launch_i4min(p, l, st);
        case WF_FP8: return mfma ? launch_mfma_fp8(p, l, st) : launch_fp8(p, l, st);
        case WF_BF16: return mfma ? launch_mfma_bf16(p, l, st) : launch_bf16(p, l, st);
        default: return BZ_ERR_INVALID_ARG;
    }
}

static bool aligned(const void* ptr, uintptr_t a) { return (reinterpret_cast<uintptr_t>(ptr) & (a - 1)) == 0; }

// Rows of x handled by one streaming launch (larger M is processed in
// slices of this many rows, each re-streaming the weights).
constexpr int kMaxRowsPerLaunch = 4;

// Workgroups the automatic launch shape aims for: about one per CU of an
// MI355X (256 CUs), each owning tiles / 256 consecutive output tiles.
constexpr int kTargetWorkgroups = 256;

// Descriptor checks shared by bz_gemv and bz_gemv_workspace; fills the
// derived sizes.
struct DescInfo {
    int n_out, glog2;
    int64_t row_bytes;
    bool i4;
};

static int check_desc(const bz_gemv_desc* d, DescInfo& di) {
    if (!d) return BZ_ERR_INVALID_ARG;
    if (d->abi_version != BZ_ABI_VERSION) return BZ_ERR_ABI;
    const int M = d->M, N = d->N, K = d->K, wf = d->wfmt, epi = d->epilogue;
    if (M < 1 || N < 1 || K < 1) return BZ_ERR_INVALID_ARG;
    if (wf < BZ_W_INT4_ZP || wf > BZ_W_FP8_TILED_PAIRED) return BZ_ERR_INVALID_ARG;
    if (epi < BZ_EPI_NONE || epi > BZ_EPI_RESIDUAL) return BZ_ERR_INVALID_ARG;
    if (d->out_dtype != BZ_DT_BF16 && d->out_dtype != BZ_DT_F32) return BZ_ERR_INVALID_ARG;
    if (!d->x || !d->w || !d->out) return BZ_ERR_INVALID_ARG;
    if (d->cfg_path < 0 || d->cfg_path > PATH_PANEL || d->cfg_slices < 0) return BZ_ERR_INVALID_ARG;
    if (d->reserved0) return BZ_ERR_INVALID_ARG;
    if (d->n_out2 && !is_tiled(wf)) return BZ_ERR_UNSUPPORTED;  // the second store is a streaming-path feature
    if (is_tiled(wf)) {
        // tiled formats: scales inside w; 16-row blocks; paired <=> SiLU-gate
        if (epi == BZ_EPI_RESIDUAL) {
            if (!d->residual) return BZ_ERR_INVALID_ARG;
            if (d->residual_dtype != BZ_DT_BF16 && d->residual_dtype != BZ_DT_F32) return BZ_ERR_INVALID_ARG;
        }
        if (tiled_paired(wf) != (epi == BZ_EPI_SILU_GATE)) return BZ_ERR_UNSUPPORTED;
        // the streaming kernel (path 5), or the several-row tile kernel (path 4)
        // or panel kernel (path 6) for unpaired weights without the second
        // store (the panel kernel also without RMSNorm)
        if (d->cfg_path == PATH_TILE || d->cfg_path == PATH_PANEL) {
            if (tiled_paired(wf) || d->n_out2) return BZ_ERR_UNSUPPORTED;
            if (d->cfg_path == PATH_PANEL && d->gamma) return BZ_ERR_UNSUPPORTED;
        } else if (d->cfg_path && d->cfg_path != PATH_STREAM) {
            return BZ_ERR_UNSUPPORTED;
        }
        if (N % 16 || !tiled_units(wf, K) || (tiled_i4(wf) && d->group != 128)) return BZ_ERR_SHAPE;
        const int n_out = epi == BZ_EPI_SILU_GATE ? N / 2 : N;
        if (d->ldx < K || d->ldo < n_out) return BZ_ERR_INVALID_ARG;
        if (epi == BZ_EPI_RESIDUAL && d->ldr < n_out) return BZ_ERR_INVALID_ARG;
        if (d->n_out2 < 0 || d->n_out2 > n_out || (d->n_out2 && (!d->out2 || d->ldo2 < d->n_out2)))
            return BZ_ERR_INVALID_ARG;
        if (!aligned(d->x, 16) || (d->ldx % 8) || !aligned(d->w, 16)) return BZ_ERR_ALIGNMENT;
        if (d->gamma && !aligned(d->gamma, 16)) return BZ_ERR_ALIGNMENT;
        if (!aligned(d->out, d->out_dtype == BZ_DT_F32 ? 4 : 2)) return BZ_ERR_ALIGNMENT;
        if (d->n_out2 && !aligned(d->out2, d->out_dtype == BZ_DT_F32 ? 4 : 2)) return BZ_ERR_ALIGNMENT;
        di.n_out = n_out;
        di.glog2 = 7;
        di.row_bytes = tiled_i4(wf) ? K / 2 : K;
        di.i4 = tiled_i4(wf);
        return BZ_OK;
    }
    if (d->cfg_path == PATH_STREAM || d->cfg_path == PATH_PANEL) return BZ_ERR_UNSUPPORTED;
    const bool i4 = (wf == BZ_W_INT4_ZP || wf == BZ_W_INT4_MIN);
    if ((i4 || wf == BZ_W_FP8) && !d->sc0) return BZ_ERR_INVALID_ARG;
    if (wf == BZ_W_INT4_MIN && !d->sc1) return BZ_ERR_INVALID_ARG;
    if (epi == BZ_EPI_RESIDUAL) {
        if (!d->residual) return BZ_ERR_INVALID_ARG;
        if (d->residual_dtype != BZ_DT_BF16 && d->residual_dtype != BZ_DT_F32) return BZ_ERR_INVALID_ARG;
    }
    if (epi == BZ_EPI_SILU_GATE && (N % 2)) return BZ_ERR_SHAPE;
    const int n_out = epi == BZ_EPI_SILU_GATE ? N / 2 : N;
    int glog2 = 0;
    int64_t row_bytes;
    if (i4) {
        const int g = d->group;
        if (g < 32 || (g & (g - 1))) return BZ_ERR_SHAPE;
        if (K % g) return BZ_ERR_SHAPE;
        while ((1 << glog2) < g) ++glog2;
        row_bytes = K / 2;
    } else if (wf == BZ_W_FP8) {
        if (K % 16) return BZ_ERR_SHAPE;
        row_bytes = K;
    } else {
        if (K % 8) return BZ_ERR_SHAPE;
        row_bytes = (int64_t)K * 2;
    }
    if (d->ldx < K || d->ldo < n_out) return BZ_ERR_INVALID_ARG;
    if (epi == BZ_EPI_RESIDUAL && d->ldr < n_out) return BZ_ERR_INVALID_ARG;
    if (!aligned(d->x, 16) || (d->ldx % 8) || !aligned(d->w, 16)) return BZ_ERR_ALIGNMENT;
    if (d->gamma && !aligned(d->gamma, 16)) return BZ_ERR_ALIGNMENT;
    if (wf == BZ_W_INT4_ZP || wf == BZ_W_FP8) {
        if (!aligned(d->sc0, 4)) return BZ_ERR_ALIGNMENT;
    } else if (wf == BZ_W_INT4_MIN) {
        if (!aligned(d->sc0, 2) || !aligned(d->sc1, 2)) return BZ_ERR_ALIGNMENT;
    }
    if (!aligned(d->out, d->out_dtype == BZ_DT_F32 ? 4 : 2)) return BZ_ERR_ALIGNMENT;
    di.n_out = n_out;
    di.glog2 = glog2;
    di.row_bytes = row_bytes;
    di.i4 = i4;
    return BZ_OK;
}

int gemv_check_desc(const bz_gemv_desc* d) {
    DescInfo di;
    return check_desc(d, di);
}

// Launch shape of the several-row tile kernel (bz_gemv_tile.h).
struct TilePlan {
    int MB, T, D, nw, ks, nsl, ncb;
    size_t lds, ws;
};

// x slice bytes the automatic rule allows per workgroup (two workgroups per
// CU fit the 160 KB of LDS), and the fewest workgroups it aims for: with 8
// waves each, measured on MI355X (C4 shapes, M = 8..32) the best slice counts
// give 160-240 workgroups; more slices only add split-K partials.
constexpr int kTileXBudget = 80 * 1024 - 512;
constexpr int kTileTargetWorkgroups = 192;

// BZ_OK and the plan of one launch over M <= kTileMaxRows rows when the tile
// kernel can run this descriptor (its cfg_* fields are read when cfg_path
// selects it); otherwise an error code.  Fewer rows never need more slices,
// LDS or workspace than more rows.
static int tile_plan(const bz_gemv_desc* d, const DescInfo& di, int M, TilePlan& pl) {
    const int K = d->K, wf = d->wfmt;
    const bool forced = d->cfg_path == PATH_TILE;
    if (d->gamma || d->epilogue == BZ_EPI_SILU_GATE) return BZ_ERR_UNSUPPORTED;
    const int UK = tile_unit_k(wf);
    if ((di.i4 && d->group < 128) || K % UK || di.row_bytes >= (1 << 24)) return BZ_ERR_UNSUPPORTED;
    // 32-bit offsets inside the kernel: x rows of a launch, a slice of partials
    if ((int64_t)M * d->ldx >= (int64_t(1) << 31) || (int64_t)tile_part_rows(M) * di.n_out * 4 >= (int64_t(1) << 31))
        return BZ_ERR_UNSUPPORTED;
    pl.MB = (M + 15) / 16;
    pl.T = forced && d->cfg_tiles ? d->cfg_tiles : 1;
    pl.D = forced && d->cfg_depth ? d->cfg_depth : 4;
    pl.nw = forced && d->cfg_waves ? d->cfg_waves : 8;
    if ((pl.T != 1 && pl.T != 2) || (pl.D != 2 && pl.D != 4 && pl.D != 8) || (pl.nw != 4 && pl.nw != 8))
        return BZ_ERR_INVALID_ARG;
    const int cbw = pl.nw * 16 * pl.T;
    pl.ncb = (di.n_out + cbw - 1) / cbw;
    if (pl.ncb > kTileCounters) return BZ_ERR_UNSUPPORTED;
    const int units = K / UK;
    int nsl;
    if (forced && d->cfg_slices) {
        nsl = d->cfg_slices;
    } else {
        const int want = (kTileTargetWorkgroups + pl.ncb - 1) / pl.ncb;
        const int max_units = std::max(1, (kTileXBudget / (2 * M) - 8) / UK);
        const int need = (units + max_units - 1) / max_units;
        nsl = std::max(want, need);
    }
    if (nsl < 1) return BZ_ERR_INVALID_ARG;
    nsl = std::min(nsl, units);
    const int upl = (units + nsl - 1) / nsl;  // units per slice
    pl.ks = upl * UK;
    pl.nsl = (units + upl - 1) / upl;
    pl.lds = (size_t)tile_lds_layout(M, pl.MB, pl.ks, wf).total;
    if (pl.lds > (size_t)device_lds_limit()) return BZ_ERR_UNSUPPORTED;
    pl.ws = pl.nsl > 1 ? kTilePartOffset + (size_t)pl.nsl * tile_part_rows(M) * di.n_out * 4 : 0;
    return BZ_OK;
}

// The automatic rule takes the tile kernel from this many rows on.
constexpr int kTileMinRows = 5;

// (Tiled formats: unpaired weights only, and not with the second store;
// not where the panel kernel is taken.)
static bool panel_auto(const bz_gemv_desc* d);
static bool stream_rows_auto(const bz_gemv_desc* d);
static bool tile_auto(const bz_gemv_desc* d) {
    return d->cfg_path == 0 && d->M >= kTileMinRows && !d->n_out2 && !tiled_paired(d->wfmt) && !panel_auto(d) &&
           !stream_rows_auto(d);
}

static int launch_tile(int wf, const TileParams& tp, const TileLaunch& l, hipStream_t st) {
    switch (wf) {
        case WF_I4ZP: return launch_tile_i4zp(tp, l, st);
        case WF_I4MIN: return launch_tile_i4min(tp, l, st);
        case WF_FP8: return launch_tile_fp8(tp, l, st);
        case WF_BF16: return launch_tile_bf16(tp, l, st);
        case BZ_W_INT4_TILED: return launch_tile_i4t(tp, l, st);
        case BZ_W_FP8_TILED: return launch_tile_f8t(tp, l, st);
        default: return BZ_ERR_INVALID_ARG;
    }
}

// Launch shape of the tiled streaming kernel for `rows` rows of x (<= 8).
// Built-in rule (sweeps of 2-16 waves on MI355X over the decode shapes at
// M = 1, 2).  With more than 256 row blocks (more workgroups than CUs):
// about 4 units (4 KiB of tiles) per wave for int4 and 6 for fp8 (int4 K2560:
// 5 waves x 4 units; fp8 K2560: 7 x 6), 8 once a row has 64 units or more.
// With at most 256 blocks each CU holds one workgroup, and shorter chains per
// wave win: 2 units per wave for rows of <= 32 units (hidden 1024-2048
// projections, int4 K4096), else 4, and from 64 units 5 for int4 (down
// K10240: 16 waves x 5) but 8 for fp8 (o_proj K4096: 13 x 5 measured
// 0.4 us slower than 8 x 8 at M = 1).  At most 16 waves.
static int stream_plan(const bz_gemv_desc* d, int rows, StreamLaunch& l) {
    const int wf = d->wfmt;
    const int NU = tiled_units(wf, d->K);
    int nw = d->cfg_waves;
    if (nw < 0 || nw > kStreamMaxWaves) return BZ_ERR_INVALID_ARG;
    const bool few_blocks = d->N / 16 <= 256;
    const int per_wave = few_blocks ? (NU <= 32 ? 2 : (NU >= 64 ? (tiled_i4(wf) ? 5 : 8) : 4))
                                    : (NU >= 64 ? 8 : (tiled_i4(wf) ? 4 : 6));
    if (!nw) nw = std::min(kStreamMaxWaves, (NU + per_wave - 1) / per_wave);
    const int need = (NU + nw - 1) / nw;
    int upw = 0;
    for (int u : kStreamUpw)
        if (u >= need) {
            upw = u;
            break;
        }
    if (!upw) return BZ_ERR_UNSUPPORTED;  // K too long for the waves
    // every wave owns at least one unit (a forced wave count above that is
    // lowered): a wave reads the staged x of its own units only
    nw = std::min(nw, (NU + upw - 1) / upw);
    l.nw = nw;
    l.upw = upw;
    l.mm = rows <= 1 ? 1 : rows <= 2 ? 2 : rows <= 4 ? 4 : 8;
    l.grid = (unsigned)(d->N / 16);
    l.lds = (size_t)stream_lds(wf, rows, d->K, nw).total;
    return l.lds <= (size_t)device_lds_limit() ? BZ_OK : BZ_ERR_UNSUPPORTED;
}

static int launch_stream(int wf, const StreamParams& p, const StreamLaunch& l, hipStream_t st) {
    switch (wf) {
        case WF_I4T: return launch_stream_i4t(p, l, st);
        case WF_I4TP: return launch_stream_i4tp(p, l, st);
        case WF_F8T: return launch_stream_f8t(p, l, st);
        case WF_F8TP: return launch_stream_f8tp(p, l, st);
        default: return BZ_ERR_INVALID_ARG;
    }
}

static int launch_wide(int wf, const StreamParams& p, const WideLaunch& l, int nblk, hipStream_t st) {
    switch (wf) {
        case WF_I4T: return launch_wide_i4t(p, l, nblk, st);
        case WF_I4TP: return launch_wide_i4tp(p, l, nblk, st);
        case WF_F8T: return launch_wide_f8t(p, l, nblk, st);
        case WF_F8TP: return launch_wide_f8tp(p, l, nblk, st);
        default: return BZ_ERR_INVALID_ARG;
    }
}

// Launch shape of the several-block kernel (bz_gemv_wide.h) for `rows` rows
// of x (<= 8) and T row blocks per workgroup.  Waves: about 2 units each for
// int4, 5 for fp8 over several blocks and 8 for fp8 over one, at most 16.
// Measured on MI355X at M = 1 (kernel time, weights rotated through 1 GiB):
// int4 gate|up K2560 N20480, 5 blocks per workgroup: 10 x 2 7.08 us, 7 x 3
// 7.06, 5 x 4 7.51; int4 qkv K2560 N6144, 2 blocks: 10 x 2 4.11, 7 x 3 4.34,
// 5 x 4 4.52; fp8 gate|up, 5 blocks: 8 x 5 10.05, 10 x 4 10.11, 7 x 6 10.75;
// fp8 o_proj K4096 N2560, 1 block: 8 x 8 4.13, 16 x 4 4.15.
static int wide_plan(const bz_gemv_desc* d, int rows, int T, WideLaunch& l) {
    l.upw = 0;  // stays 0 when no unit count fits (the caller tells that apart from an LDS overflow)
    const int wf = d->wfmt;
    const int NU = tiled_units(wf, d->K), nblk = d->N / 16;
    if (T < 1 || T > kWideMaxBlocks) return BZ_ERR_INVALID_ARG;
    int nw = d->cfg_waves;
    if (nw < 0 || nw > kStreamMaxWaves) return BZ_ERR_INVALID_ARG;
    const int mm = rows <= 1 ? 1 : rows <= 2 ? 2 : rows <= 4 ? 4 : 8;
    // units per wave: int4 2, or 4 over more than 20 units with more than 2
    // rows (int4 K4096 N2560 M = 5: 8 waves x 4 units 4.51 us, 16 x 2 4.74+);
    // fp8 5 over several blocks, 8 over one
    const int per_wave = tiled_i4(wf) ? (mm > 2 && NU > 20 ? 4 : 2) : T > 1 ? 5 : 8;
    if (!nw) nw = std::min(kStreamMaxWaves, (NU + per_wave - 1) / per_wave);
    const int need = (NU + nw - 1) / nw;
    int upw = 0;
    for (int u : kWideUpw)
        if (u >= need && u <= wide_max_upw(wf, 1)) {
            upw = u;
            break;
        }
    if (!upw) return BZ_ERR_UNSUPPORTED;  // K too long for the waves
    l.upw = upw;
    if (upw > wide_max_upw(wf, mm)) return BZ_ERR_UNSUPPORTED;  // fits over fewer rows of x
    nw = std::min(nw, (NU + upw - 1) / upw);  // every wave owns at least one unit
    l.nw = nw;
    l.mm = mm;
    l.T = T;
    l.grid = (unsigned)((nblk + T - 1) / T);
    l.lds = (size_t)wide_lds(wf, rows, d->K, T).total;
    return l.lds <= (size_t)device_lds_limit() ? BZ_OK : BZ_ERR_UNSUPPORTED;
}

// Row blocks per workgroup the rule gives the several-block kernel, 0 for
// the one-block streaming kernel:
//   * more row blocks than the 256 CUs: enough blocks per workgroup for one
//     workgroup per CU (gate|up N = 20480: 5; qkv N = 6144: 2).  Measured on
//     MI355X at M = 1 against the one-block kernel: int4 gate|up 7.59 ->
//     7.08 us, int4 qkv 4.54 -> 4.11 us, fp8 gate|up 10.52 -> 10.05 us;
//   * fp8 rows of 64 units or more (K >= 4096) over at most 256 blocks: one
//     block per workgroup, all its tiles in flight behind the x loads (fp8
//     down K10240 N2560 7.43 -> 7.18 us, fp8 o_proj K4096 N2560 4.38 -> 4.13).
//     Not fp8 qkv K2560 N4096 (one-block 3.92 us, several-block 4.02) nor the
//     int4 rows of at most 256 blocks (int4 down K10240 N2560 5.69 against
//     5.74, o_proj K4096 3.77 both);
//   * 3 to 8 rows over rows of at most kWideShortK (one launch), unpaired and
//     without RMSNorm (the cases measured): one block per workgroup where
//     that plan fits.  At M = 3 / 4, against the one-block
//     kernel: int4 K4096 N2560 4.21 / 4.40 -> 4.05 / 4.17 us, int4 K2560
//     N4096 4.02 / 4.22 -> 3.90 / 3.98, fp8 K2560 N4096 4.38 / 4.41 -> 4.12
//     / 4.18, fp8 K2048 N2048 3.57 / 3.71 -> 3.38 / 3.46 (int4 K2048 N2048
//     3.36 / 3.49 -> 3.38 / 3.59: within the noise at the M = 3 it mostly
//     sees); int4 K6144 N2048 (+ residual) M = 4 5.19 -> 5.00.  At M = 5-8 see
//     stream_rows_auto.
constexpr int kWideShortK = 8192;
static int wide_rule(const bz_gemv_desc* d, int rows) {
    const int nblk = d->N / 16, NU = tiled_units(d->wfmt, d->K);
    if (nblk > 256) return std::min(kWideMaxBlocks, (nblk + 255) / 256);
    if (!tiled_i4(d->wfmt) && NU >= 64) return 1;
    if (rows >= 3 && d->K <= kWideShortK && !tiled_paired(d->wfmt) && !d->gamma) {
        WideLaunch w{};
        if (wide_plan(d, rows, 1, w) == BZ_OK) return 1;
    }
    return 0;
}

// The streaming kernel a tiled descriptor runs on and its launch shape: the
// rule's choice without a cfg; on path 5 forced, cfg_tiles = 0 the one-block
// kernel and cfg_tiles >= 1 the several-block kernel with that many blocks
// per workgroup (cfg_waves waves, 0 = the kernel's own rule, either way).
struct TiledPlan {
    bool wide;
    StreamLaunch s;
    WideLaunch w;
};

static int tiled_plan(const bz_gemv_desc* d, int rows, TiledPlan& pl) {
    int T;
    if (d->cfg_path == PATH_STREAM) {
        if (d->cfg_tiles < 0 || d->cfg_tiles > kWideMaxBlocks) return BZ_ERR_INVALID_ARG;
        T = d->cfg_tiles;
    } else {
        T = wide_rule(d, rows);
        // a row too long for the several-block kernel's waves (int4 beyond
        // 16 x 5 units) stays on the one-block kernel
        if (T && wide_plan(d, rows, T, pl.w) == BZ_ERR_UNSUPPORTED && pl.w.upw == 0) T = 0;
    }
    pl.wide = T > 0;
    return pl.wide ? wide_plan(d, rows, T, pl.w) : stream_plan(d, rows, pl.s);
}

// The tiled formats: up to kStreamMaxRows rows per launch (fewer when their
// staged x does not fit the LDS), each launch streaming the weights once.
static int gemv_tiled(const bz_gemv_desc* d, const DescInfo& di, hipStream_t st) {
    const int M = d->M;
    int rows = std::min(M, kStreamMaxRows);
    TiledPlan pl{};
    int rc = tiled_plan(d, rows, pl);
    while (rc == BZ_ERR_UNSUPPORTED && rows > 1 && (pl.wide ? pl.w.upw : pl.s.upw)) rc = tiled_plan(d, --rows, pl);
    if (rc != BZ_OK) return rc;
    TiledPlan pl_rem = pl;  // the last, shorter launch (planned before anything is launched)
    if (M > rows && M % rows && tiled_plan(d, M % rows, pl_rem) != BZ_OK) return BZ_ERR_UNSUPPORTED;
    StreamParams p{};
    p.ldx = d->ldx;
    p.w = static_cast<const uint8_t*>(d->w);
    p.chunk = tiled_chunk_bytes(d->wfmt, tiled_units(d->wfmt, d->K));
    p.gamma = static_cast<const uint16_t*>(d->gamma);
    p.ldr = d->ldr;
    p.ldo = d->ldo;
    p.ldo2 = d->ldo2;
    p.n_out2 = d->n_out2;
    p.eps = d->eps;
    p.K = d->K;
    p.NU = tiled_units(d->wfmt, d->K);
    p.n_out = di.n_out;
    p.epi = d->epilogue;
    p.out_f32 = d->out_dtype == BZ_DT_F32;
    p.res_f32 = d->residual_dtype == BZ_DT_F32;
    p.norm = d->gamma != nullptr;
    p.x_lead = p.NU >= 80 && d->N / 16 <= 256;
    const size_t osz = p.out_f32 ? 4 : 2, rsz = p.res_f32 ? 4 : 2;
    for (int m0 = 0; m0 < M; m0 += rows) {
        const int r = std::min(rows, M - m0);
        const TiledPlan& q = r == rows ? pl : pl_rem;
        p.M = r;
        p.x = static_cast<const uint16_t*>(d->x) + (int64_t)m0 * d->ldx;
        p.out = static_cast<uint8_t*>(d->out) + (int64_t)m0 * d->ldo * osz;
        p.out2 = d->n_out2 ? static_cast<uint8_t*>(d->out2) + (int64_t)m0 * d->ldo2 * osz : nullptr;
        p.res = d->residual ? static_cast<const uint8_t*>(d->residual) + (int64_t)m0 * d->ldr * rsz : nullptr;
        const int lrc = q.wide ? launch_wide(d->wfmt, p, q.w, d->N / 16, st) : launch_stream(d->wfmt, p, q.s, st);
        if (lrc != BZ_OK) return lrc;
    }
    return BZ_OK;
}

// Row blocks per workgroup of the panel kernel's automatic rule: every
// workgroup reads all of x for its blocks, so a workgroup takes as many
// blocks as keep the grid at one workgroup per CU (256), at most 5.
static int panel_blocks(int nblk) { return std::min(5, std::max(1, (nblk + 255) / 256)); }

// Descriptors the panel kernel can run: unpaired tiled weights without
// RMSNorm or the second store.
static bool panel_ok(const bz_gemv_desc* d) {
    return is_tiled(d->wfmt) && !tiled_paired(d->wfmt) && !d->gamma && !d->n_out2;
}

// The automatic rule takes the panel kernel for them (measured on MI355X
// against the streaming and tile kernels, int4 and fp8, N = 1024-20480,
// K = 2560-10240, M = 2..32):
//   * from 5 rows on, with K slices for rows of at least kPanelSliceMinK
//     when the x of a launch exceeds kPanelSliceX or the weight has fewer
//     than kPanelSliceFewBlocks row blocks, and the workspace they need is
//     given (else over the whole K);
//   * but not for 5-8 rows over rows of at most kWideShortK, which the
//     several-block streaming kernel runs in one launch (stream_rows_auto).
static bool panel_auto(const bz_gemv_desc* d) {
    if (d->cfg_path || !panel_ok(d)) return false;
    return d->M >= 5 && !stream_rows_auto(d);
}

// 5 to 8 rows of x over rows of at most kWideShortK: the streaming kernels
// (wide_rule) in one launch, not the panel or tile kernel.  Measured on
// MI355X (graph replays over >= 1 GiB of copies, us, M = 5 / 8; the panel
// kernel's whole-K plan, then the several-block kernel):
//   int4 K4096 N2560 5.61 / 5.62 -> 4.51 / 4.94, fp8 4.46 / 5.63 -> 4.55 / 4.69;
//   int4 K2560 N4096 4.78 / 4.80 -> 4.29 / 4.75, fp8 5.32 / 5.07 -> 4.46 / 4.55;
//   int4 K2560 N6144 6.46 / 6.44 -> 5.10 / 5.69, fp8 7.21 / 6.43 -> 5.13 / 5.17;
//   int4 K2560 N20480 9.58 / 8.92 -> 8.18 / 8.95, fp8 11.33 / 10.83 -> 10.57 / 10.90;
//   fp8 K2048 N2048 4.65 / 4.66 -> 3.60 / 3.60 (4 waves).
//   and up to K8192, against the panel kernel (+ residual, M = 8): int4 K6144
//   N2048 7.26 -> 6.01, fp8 K8192 N1024 (over 4 K slices) 7.72 -> 6.00.
// Over K10240 the panel kernel's K slices win (fp8 M = 8: 10.23 against the
// several-block kernel's 16 waves x 10 units; int4 does not fit the waves
// at 8 rows).  Only where the several-block plan runs all the rows in one
// launch.  From 9 rows on the streaming kernels need two launches and the
// panel kernel wins (int4 K4096 N2560 M = 12: 5.64 against 9.03).  The same
// 3-4 rows of fp8 over 1280 blocks went to the panel kernel before: the
// several-block kernel is faster there too (K2560 N20480 M = 3 / 4: 10.17 /
// 10.28 against 10.3+ / 10.71).
static bool stream_rows_auto(const bz_gemv_desc* d) {
    if (d->cfg_path != 0 || !panel_ok(d) || d->M < kTileMinRows || d->M > kStreamMaxRows || d->K > kWideShortK)
        return false;
    const int T = wide_rule(d, d->M);
    WideLaunch w{};
    return T > 0 && wide_plan(d, d->M, T, w) == BZ_OK;
}

// x bytes of one launch above which the automatic rule splits K into slices
// (every workgroup reads all of x over its K range from L2), the shortest
// rows it splits, the most row blocks per workgroup it takes then (int4,
// fp8; fewer for small N: one per kPanelSliceBlockRows blocks) and the
// workgroups the slice count aims for.  Measured on MI355X (graph replays
// over >= 1 GiB of weight copies, us):
//   K10240 N2560, against the whole K and the tile kernel's 128-column
//   blocks over 8-10 slices: int4 M = 32 2 blocks x 3 slices 12.7 (whole K
//   13.9, tile 13.4), M = 16 2 x 2 9.75 (10.0, 10.5), M = 12 2 x 3 8.80
//   (9.26); fp8 M = 32 3 x 4 13.2 (tile 15.4), M = 16 3 x 4 10.6 (whole K
//   12.0), M = 12 3 x 4 10.1 (11.4), M = 8 3 x 4 9.81 (10.24);
//   K8192 N1024 (64 blocks), sliced at every M since the whole K fills only
//   64 CUs: fp8 M = 5 1 x 4 7.15 (whole K 7.61), M = 8 1 x 4 7.18 (7.94),
//   M = 16 1 x 4 7.31 (9.51), M = 32 1 x 4 8.39 (3 x 11: 11.48); int4 M = 5
//   1 x 4 7.02 (7.74), M = 8 7.08 (7.78), M = 16 1 x 4 7.06 (8.50), M = 32
//   1 x 4 8.27 (3 x 11: 10.31);
//   not for K <= 4096: K4096 N2560 and K2560 N4096 / N6144 at M = 16, 32
//   run as fast or faster over the whole K (fp8 K4096 M = 32 8.10 against
//   8.29 over 2 x 3).
constexpr int64_t kPanelSliceX = 128 * 1024;
constexpr int kPanelSliceMinK = 8192;
constexpr int kPanelSliceBlocksI4 = 2, kPanelSliceBlocksF8 = 3;
constexpr int kPanelSliceBlockRows = 48;
constexpr int kPanelSliceFewBlocks = 128;  // fewer blocks: slices whatever the x bytes
constexpr int kPanelTargetWorkgroups = 240;

// Launch shape of the panel kernel (bz_gemv_panel.h) for `rows` <= 32 rows
// of x: nsl K slices (cfg_slices; by default 1, or about
// kPanelTargetWorkgroups workgroups in all where the rule above slices K and
// that makes at least 2), T row blocks per workgroup (cfg_tiles: 1 to 5;
// default by the number of blocks, or with the rule's slices
// kPanelSliceBlocks* or fewer), NW waves (cfg_waves; default about 5 units
// per wave, 4 over K slices and at least 8 over slices of one block; at most
// 16 waves, 8 with several blocks) splitting the slice's units UPW each.
// `slices` > 0 overrides both the cfg and the rule (1: no workspace).
static int panel_plan(const bz_gemv_desc* d, int rows, PanelLaunch& l, int slices = 0) {
    const int wf = d->wfmt;
    if (tiled_paired(wf) || d->gamma || d->n_out2) return BZ_ERR_UNSUPPORTED;
    const int NU = tiled_units(wf, d->K);
    if (!NU) return BZ_ERR_SHAPE;
    if ((int64_t)rows * d->ldx * 2 >= (int64_t(1) << 31)) return BZ_ERR_UNSUPPORTED;  // 32-bit x offsets
    const int nblk = d->N / 16;
    if (d->cfg_slices < 0) return BZ_ERR_INVALID_ARG;
    int nsl = slices ? slices : d->cfg_slices;
    const int slice_blocks =
        std::max(1, std::min(tiled_i4(wf) ? kPanelSliceBlocksI4 : kPanelSliceBlocksF8, nblk / kPanelSliceBlockRows));
    const int slice_groups = (nblk + slice_blocks - 1) / slice_blocks;
    const bool rule_slices = !nsl && d->K >= kPanelSliceMinK &&
                             ((int64_t)rows * d->K * 2 > kPanelSliceX || nblk < kPanelSliceFewBlocks) &&
                             (kPanelTargetWorkgroups + slice_groups / 2) / slice_groups >= 2;
    const int T = d->cfg_tiles                 ? d->cfg_tiles
                  : rule_slices || nsl > 1 ? slice_blocks
                                           : panel_blocks(nblk);
    bool t_ok = false;
    for (int t : kPanelBlocks) t_ok |= t == T;
    if (!t_ok) return BZ_ERR_INVALID_ARG;
    const int groups = (nblk + T - 1) / T;
    if (rule_slices) nsl = std::max(1, (kPanelTargetWorkgroups + groups / 2) / groups);
    if (!nsl) nsl = 1;
    nsl = std::min(nsl, NU);
    const int ups = (NU + nsl - 1) / nsl;
    nsl = (NU + ups - 1) / ups;
    if (nsl > 1 && (groups > kTileCounters || (int64_t)nsl * rows * nblk * 16 * 4 >= (int64_t(1) << 31)))
        return BZ_ERR_UNSUPPORTED;
    const int maxw = T == 1 ? kPanelMaxWaves : 8;
    int nw = d->cfg_waves;
    if (nw < 0 || nw > maxw) return BZ_ERR_INVALID_ARG;
    // sliced: int4 K10240 M = 16 7 waves x 4 units 9.25 us, 6 x 5 9.78; one
    // block over K8192 slices of 16 units: int4 M = 32 8 x 2 8.27, 4 x 4 8.6+
    if (!nw) nw = std::min(maxw, nsl > 1 ? std::max((ups + 3) / 4, T == 1 ? 8 : 1) : (ups + 4) / 5);
    const int need = (ups + nw - 1) / nw;
    int upw = 0;
    for (int u : kPanelUpw)
        if (u >= need) {
            upw = u;
            break;
        }
    if (!upw) return BZ_ERR_UNSUPPORTED;  // K too long for the waves
    l.nw = (ups + upw - 1) / upw;         // every wave owns at least one unit
    l.upw = upw;
    l.T = T;
    l.mt = rows > 16 ? 2 : 1;
    l.nsl = nsl;
    l.ups = ups;
    l.grid = (unsigned)(groups * nsl);
    l.lds = (size_t)panel_lds(l.nw, T, l.mt);
    l.ws = nsl > 1 ? kTilePartOffset + (size_t)nsl * rows * nblk * 16 * 4 : 0;
    return l.lds <= (size_t)device_lds_limit() ? BZ_OK : BZ_ERR_UNSUPPORTED;
}

// Whether a descriptor's workspace holds `ws` bytes (16-byte aligned).
static bool workspace_holds(const bz_gemv_desc* d, size_t ws) {
    return !ws || (d->workspace && aligned(d->workspace, 16) && d->workspace_bytes >= ws);
}

// The panel plan of `rows` rows the call can run: the one asked for, or,
// chosen by the rule but without the workspace its K slices need, the
// whole-K plan.
static int panel_plan_call(const bz_gemv_desc* d, int rows, PanelLaunch& l) {
    int rc = panel_plan(d, rows, l);
    if (rc != BZ_OK || workspace_holds(d, l.ws)) return rc;
    if (d->cfg_path == PATH_PANEL && d->cfg_slices) return BZ_ERR_INVALID_ARG;  // forced slices, no workspace
    return panel_plan(d, rows, l, 1);
}

// The panel kernel over all M rows, kPanelMaxRows per launch.
static int gemv_panel_rows(const bz_gemv_desc* d, hipStream_t st) {
    const int M = d->M;
    const int rows = std::min(M, kPanelMaxRows);
    PanelLaunch l{}, l_rem{};
    int rc = panel_plan_call(d, rows, l);
    if (rc != BZ_OK) return rc;
    if (M > rows && M % rows && (rc = panel_plan_call(d, M % rows, l_rem)) != BZ_OK) return rc;
    PanelParams p{};
    p.ldx = d->ldx;
    p.w = static_cast<const uint8_t*>(d->w);
    p.NU = tiled_units(d->wfmt, d->K);
    p.chunk = tiled_chunk_bytes(d->wfmt, p.NU);
    p.ldr = d->ldr;
    p.ldo = d->ldo;
    p.K = d->K;
    p.nblk = d->N / 16;
    p.epi = d->epilogue;
    p.out_f32 = d->out_dtype == BZ_DT_F32;
    p.res_f32 = d->residual_dtype == BZ_DT_F32;
    p.cnt = static_cast<uint32_t*>(d->workspace);
    p.part = d->workspace ? reinterpret_cast<float*>(static_cast<uint8_t*>(d->workspace) + kTilePartOffset) : nullptr;
    const size_t osz = p.out_f32 ? 4 : 2, rsz = p.res_f32 ? 4 : 2;
    for (int m0 = 0; m0 < M; m0 += rows) {
        const int r = std::min(rows, M - m0);
        const PanelLaunch& q = r == rows ? l : l_rem;
        p.M = r;
        p.nsl = q.nsl;
        p.ups = q.ups;
        p.x = static_cast<const uint16_t*>(d->x) + (int64_t)m0 * d->ldx;
        p.out = static_cast<uint8_t*>(d->out) + (int64_t)m0 * d->ldo * osz;
        p.res = d->residual ? static_cast<const uint8_t*>(d->residual) + (int64_t)m0 * d->ldr * rsz : nullptr;
        const int lrc = d->wfmt == WF_I4T ? launch_panel_i4t(p, q, st) : launch_panel_f8t(p, q, st);
        if (lrc != BZ_OK) return lrc;
    }
    return BZ_OK;
}

}  // namespace bz

using namespace bz;

extern "C" size_t bz_gemv_workspace(const bz_gemv_desc* d) {
    DescInfo di;
    if (check_desc(d, di) != BZ_OK) return 0;
    if (d->cfg_path == PATH_PANEL || panel_auto(d)) {
        PanelLaunch l{};
        return panel_plan(d, std::min(d->M, kPanelMaxRows), l) == BZ_OK ? l.ws : 0;
    }
    if (d->cfg_path != PATH_TILE && !tile_auto(d)) return 0;
    TilePlan pl{};
    return tile_plan(d, di, std::min(d->M, kTileMaxRows), pl) == BZ_OK ? pl.ws : 0;
}

extern "C" int bz_gemv(const bz_gemv_desc* d, void* stream) {
    DescInfo di;
    const int rc0 = check_desc(d, di);
    if (rc0 != BZ_OK) return rc0;
    const int M = d->M, N = d->N, K = d->K, wf = d->wfmt, epi = d->epilogue;
    const bool tiled = is_tiled(wf);
    const int n_out = di.n_out, glog2 = di.glog2;
    const int64_t row_bytes = di.row_bytes;
    const bool i4 = di.i4;

    if (d->cfg_path == PATH_PANEL || panel_auto(d)) return gemv_panel_rows(d, static_cast<hipStream_t>(stream));

    // several-row tile kernel (forced, or automatic from kTileMinRows rows on
    // when the caller passed the workspace it needs): kTileMaxRows rows per
    // launch
    if (d->cfg_path == PATH_TILE || tile_auto(d)) {
        TilePlan pl{};
        const int trc = tile_plan(d, di, std::min(M, kTileMaxRows), pl);
        bool ws_ok = pl.ws == 0;
        if (trc == BZ_OK && pl.ws)
            ws_ok = d->workspace && aligned(d->workspace, 16) && d->workspace_bytes >= pl.ws;
        if (d->cfg_path == PATH_TILE) {
            if (trc != BZ_OK) return trc;
            if (!ws_ok) return BZ_ERR_INVALID_ARG;
        }
        if (trc == BZ_OK && ws_ok) {
            TileParams tp{};
            GemvParams& p = tp.p;
            p.w = static_cast<const uint8_t*>(d->w);
            p.row_bytes = row_bytes;
            p.sc0 = d->sc0;
            p.sc1 = d->sc1;
            p.gamma = nullptr;
            p.ldx = d->ldx;
            p.ldr = d->ldr;
            p.ldo = d->ldo;
            p.eps = d->eps;
            p.N = N;
            p.K = K;
            p.G = i4 ? K / d->group : 0;
            p.glog2 = glog2;
            p.n_out = n_out;
            p.nchunks = 0;
            p.ntiles = 0;
            p.tpw = 0;
            p.epi = epi;
            p.out_f32 = d->out_dtype == BZ_DT_F32;
            p.res_f32 = d->residual_dtype == BZ_DT_F32;
            p.norm = 0;
            tp.cnt = static_cast<uint32_t*>(d->workspace);
            tp.NU = tiled ? tiled_units(wf, K) : 0;
            tp.chunk = tiled ? (int64_t)tiled_chunk_bytes(wf, tp.NU) : 0;
            // the plan of a last, shorter launch (checked before anything is launched)
            TilePlan pl_rem = pl;
            if (M > kTileMaxRows && M % kTileMaxRows && tile_plan(d, di, M % kTileMaxRows, pl_rem) != BZ_OK)
                return BZ_ERR_UNSUPPORTED;
            const size_t osz = p.out_f32 ? 4 : 2, rsz = p.res_f32 ? 4 : 2;
            hipStream_t st = static_cast<hipStream_t>(stream);
            for (int m0 = 0; m0 < M; m0 += kTileMaxRows) {
                const int rows = std::min(M - m0, kTileMaxRows);
                const TilePlan& q = rows == std::min(M, kTileMaxRows) ? pl : pl_rem;
                p.x = static_cast<const uint16_t*>(d->x) + (int64_t)m0 * d->ldx;
                p.out = static_cast<uint8_t*>(d->out) + (int64_t)m0 * d->ldo * osz;
                p.res = d->residual ? static_cast<const uint8_t*>(d->residual) + (int64_t)m0 * d->ldr * rsz : nullptr;
                tp.M = rows;
                tp.ks = q.ks;
                tp.nsl = q.nsl;
                tp.part = q.ws ? reinterpret_cast<float*>(static_cast<uint8_t*>(d->workspace) + kTilePartOffset)
                               : nullptr;
                TileLaunch l;
                l.MB = q.MB;
                l.T = q.T;
                l.D = q.D;
                l.nw = q.nw;
                l.lds = q.lds;
                l.grid = (unsigned)(q.ncb * q.nsl);
                const int rc = launch_tile(wf, tp, l, st);
                if (rc != BZ_OK) return rc;
            }
            return BZ_OK;
        }
    }
    if (tiled) return gemv_tiled(d, di, static_cast<hipStream_t>(stream));

    const bool silu = epi == BZ_EPI_SILU_GATE;
    const int T = silu ? 2 : 1;
    // Paths: the matrix-core kernels need 64-byte units that hold one int4
    // group (group >= 128); the int8 one also whole units (K % 128 == 0).
    const bool mfma_ok = !i4 || d->group >= 128;
    const bool i8_ok = i4 && d->group >= 128 && K % 128 == 0;
    if ((d->cfg_path == 2 && !mfma_ok) || (d->cfg_path == 3 && !i8_ok)) return BZ_ERR_UNSUPPORTED;
    // Automatic choice (measured on MI355X, M = 1..16): the int8 matrix-core
    // path for several rows over short rows (K <= 4096: every workgroup
    // stages all of x, 2 bytes per element, which long rows make costly);
    // the dot2 kernel for a single-row SiLU-gate pair; the bf16 matrix-core
    // path otherwise.
    const int path = d->cfg_path                          ? d->cfg_path
                     : (i8_ok && M > 1 && K <= 4096)      ? PATH_I8
                     : (mfma_ok && !(silu && M == 1))     ? PATH_MFMA
                                                           : PATH_DOT2;
    const bool mfma = path != PATH_DOT2;
    const int cols_per_tile = mfma ? 16 : 8;
    const int unit_bytes = mfma ? 64 : 128;
    const int nunits = (int)((row_bytes + unit_bytes - 1) / unit_bytes);
    const int ntiles = (n_out + cols_per_tile - 1) / cols_per_tile;
    Launch l;
    l.silu = silu;
    l.nw = d->cfg_waves ? d->cfg_waves : (nunits > kMaxWaves ? kMaxWaves : nunits);
    if (l.nw < 1 || l.nw > kMaxWaves) return BZ_ERR_INVALID_ARG;
    if (l.nw > nunits) l.nw = nunits;  // every wave owns at least one unit of each tile
    // Workgroups: one per cfg_tiles tiles, or ceil(ntiles / 256) tiles each
    // (about one workgroup per CU); each takes a balanced share of the tiles
    // (tpw = the largest share).
    if (d->cfg_tiles < 0) return BZ_ERR_INVALID_ARG;
    const int want = d->cfg_tiles ? d->cfg_tiles : (ntiles + kTargetWorkgroups - 1) / kTargetWorkgroups;
    const int grid = (ntiles + want - 1) / want;
    const int tpw = (ntiles + grid - 1) / grid;
    l.grid = (unsigned)grid;
    if (d->cfg_depth && ((d->cfg_depth != 2 && d->cfg_depth != 4 && d->cfg_depth != 8 && d->cfg_depth != 16) ||
                         d->cfg_depth * T > kMaxLoadsInFlight || (path == PATH_I8 && d->cfg_depth > 8)))
        return BZ_ERR_INVALID_ARG;
    // (argument validation ends here: the rest may query the device)
    // Measured on MI355X: 8 waves with 2 steps in flight per wave for a
    // SiLU-gate pair (each step loads two tiles) and 4 for single tiles on
    // the matrix-core paths; deeper pipelines only lengthen the queue the x
    // loads wait in.
    l.depth = d->cfg_depth ? d->cfg_depth : (T == 1 && (path != PATH_DOT2 || wf == BZ_W_BF16) ? 4 : 2);
    const int lds_lim = device_lds_limit();
    const int nchunks = (int)((row_bytes + 127) / 128);

    GemvParams p;
    p.w = static_cast<const uint8_t*>(d->w);
    p.row_bytes = row_bytes;
    p.sc0 = d->sc0;
    p.sc1 = d->sc1;
    p.gamma = static_cast<const uint16_t*>(d->gamma);
    p.eps = d->eps;
    p.ldx = d->ldx;
    p.ldr = d->ldr;
    p.ldo = d->ldo;
    p.N = N;
    p.K = K;
    p.G = i4 ? K / d->group : 0;
    p.glog2 = glog2;
    p.n_out = n_out;
    p.nchunks = nchunks;
    p.ntiles = ntiles;
    p.tpw = tpw;
    p.epi = epi;
    p.out_f32 = d->out_dtype == BZ_DT_F32;
    p.res_f32 = d->residual_dtype == BZ_DT_F32;
    p.norm = d->gamma != nullptr;
    hipStream_t st = static_cast<hipStream_t>(stream);
    const size_t osz = p.out_f32 ? 4 : 2, rsz = p.res_f32 ? 4 : 2;
    // rows per launch: 4 on the bf16 paths; up to the 16 rows of the MFMA A
    // operand on the int8 path, as many as its LDS (2 bytes of x per
    // element) allows
    const int rows = path == PATH_I8 ? i8_max_rows(K, lds_lim, T, l.nw, tpw) : kMaxRowsPerLaunch;
    if (rows < 1) return BZ_ERR_UNSUPPORTED;
    for (int m0 = 0; m0 < M; m0 += rows) {
        l.M = (M - m0) < rows ? (M - m0) : rows;
        const int lds = path == PATH_I8 ? i8_lds_layout(l.M, T, l.nw, K, tpw).total
                        : mfma          ? mfma_lds_layout(l.M, T, l.nw, K, wf, tpw).total
                                        : lds_layout(l.M, T, l.nw, K, wf, tpw).total;
        if (lds > lds_lim) return BZ_ERR_UNSUPPORTED;
        l.lds = (size_t)lds;
        p.x = static_cast<const uint16_t*>(d->x) + (int64_t)m0 * d->ldx;
        p.out = static_cast<uint8_t*>(d->out) + (int64_t)m0 * d->ldo * osz;
        p.res = d->residual ? static_cast<const uint8_t*>(d->residual) + (int64_t)m0 * d->ldr * rsz : nullptr;
        const int rc = launch_wf(wf, path, p, l, st);
        if (rc != BZ_OK) return rc;
    }
    return BZ_OK;
}
