// Host side of the GEMM family: argument checks, tile-shape heuristic, launch.
//
// Replaces the reference's launch_fp8_gemm / launch_fp4_gemm / launch_fp8_dequant_gemm /
// launch_bf16_gemm (csrc/jit_kernels/fp8_gemm.hpp:11-151, fp8_dequant_gemm.hpp:24-95,
// bf16_gemm.hpp:16-78) and its select_gemm_config cost model
// (csrc/jit_kernels/heuristics.hpp:592-755).  Kernels are compiled ahead of time for a
// fixed menu of tile shapes; the heuristic scores each shape with a gfx950 model
// (256 CUs, waves-of-tiles quantisation, measured cycles per K stage of each tile shape and a
// fixed per-tile cost) and memoises the choice per problem signature.
#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <tuple>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "gemm_tiles.hpp"
#include "../../include/deep_gemm_amd.h"

namespace {

thread_local std::string g_last_error;

}  // namespace

extern "C" __attribute__((visibility("hidden"))) int dg_set_error(const char* msg) {
    g_last_error = msg;
    return DG_EINVAL;
}

extern "C" const char* dg_last_error(void) { return g_last_error.c_str(); }

extern "C" const char* dg_version(void) { return "deep_gemm_amd 0.1.0 (gfx950)"; }

extern "C" int dg_device_num_cus(int32_t device) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess) {
        dg_set_error("hipDeviceGetAttribute(MultiprocessorCount) failed");
        return DG_ELAUNCH;
    }
    return n;
}

namespace dg {

// csrc/status.hip: m_indices layout check of M-grouped launches (reports through the sticky error
// words; with may_alloc false it never allocates them)
int check_m_indices(const int32_t* idx, int m, int alignment, int num_groups, hipStream_t st, bool may_alloc,
                    int32_t* blk_end = nullptr);
// csrc/status.hip: the run table of an m_indices layout (for anchored tiles)
int m_indices_runs(const int32_t* idx, int m, int alignment, int32_t* runs, const int32_t* blk_end, hipStream_t st);

KernelFn lookup_kernel(int kind, int bm, int bn, int epi, bool persistent) {
    switch (kind) {
        case kFP8FP8: return lookup_kernel_fp8fp8(bm, bn, epi, persistent);
        case kFP8FP4: return lookup_kernel_fp8fp4(bm, bn, epi, persistent);
        case kFP4FP4: return lookup_kernel_fp4fp4(bm, bn, epi, persistent);
        case kBF16: return lookup_kernel_bf16(bm, bn, epi, persistent);
        default: return nullptr;
    }
}

KernelFn lookup_walk(int kind, int bm, int bn, int epi) {
    switch (kind) {
        case kFP8FP8: return lookup_walk_fp8fp8(bm, bn, epi);
        case kBF16: return lookup_walk_bf16(bm, bn, epi);
        default: return nullptr;
    }
}

int device_cus() {
    static int cached[64] = {0};
    int dev = 0;
    (void)hipGetDevice(&dev);
    if (dev < 0 || dev >= 64) return 256;
    if (cached[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cached[dev] = n;
    }
    return cached[dev];
}

// Tiles taller than 256 rows serve M-grouped layouts only, anchored at each group's (psum) or run's
// (m_indices) first row (gemm_kernel.hpp, anchored_tile); there BM need not divide the alignment.
bool tile_anchored(int bm) { return bm > 256; }

bool tile_allowed(const dg_gemm_args& a, int bm, int bn) {
    (void)bn;
    if (tile_anchored(bm)) return a.gemm_type == kMGroupedPsum || a.gemm_type == kMGroupedIdx;
    if (a.gemm_type == kMGroupedPsum || a.gemm_type == kMGroupedIdx) {
        if (a.alignment % bm != 0) return false;
    }
    return true;
}

// Launch plan: tile shape and K split.
struct Plan {
    TileCfg tile;
    int split;          // K ranges per tile (1 = no split)
    int split_stages;   // K stages per range (skinny kernel: 64-K blocks per range)
    int skinny_nw;      // > 0: the skinny-M kernel with this many waves (tile = 32 mt x 32 nb)
    int skinny_d;       // its ring depth
    int skinny_ar;      // and rows of A it stages
    int skinny_rows;    // 1: the shared-ring decode kernel (skinny_rows_kernel, skinny_nw = mt x nb waves, ring skinny_d)
    int gemv_mr;        // > 0: the decode GEMV kernel for M <= gemv_mr (split_stages = rows of B per wave)
    int split_reduce;   // 1: split-K partials summed by a second launch (shared-ring kernel only)
};

// K elements of one kernel stage of tile t
int k_stage_elems(int kind, const TileCfg& t) { return (kind == kBF16 ? 32 : 64) * std::max(1, t.km); }

// Split-K is offered to dense / batched GEMMs whose tiles alone cannot fill the CUs.
bool split_capable(const dg_gemm_args& a) { return a.gemm_type == kNormal || a.gemm_type == kBatched; }

int64_t plan_tiles(const dg_gemm_args& a, const TileCfg& t) {
    const int groups = (a.gemm_type == kBatched || a.gemm_type == kMasked || a.gemm_type == kKGrouped) ? a.num_groups : 1;
    // anchored tiles: each group's rows start a new tile, so at most one extra tile row per group
    const int64_t mrows = ceil_div(a.m, t.bm) + (!tile_anchored(t.bm) ? 0
                                                 : a.gemm_type == kMGroupedIdx ? ceil_div(a.m, std::max(1, a.alignment))
                                                                               : a.num_groups);
    return mrows * ceil_div(a.n, t.bn) * groups;
}

// Workspace layout: a fixed area of tile counters that every launch leaves at zero (shared by
// all plans, so a partial tile of one plan never lands on another plan's counters), then the
// partial tiles.
constexpr int64_t kCounterBytes = 64 * 1024;
constexpr int kXcds = 8;   // MI355X: 8 XCDs, workgroup b dispatched to XCD b % 8
constexpr int64_t kMaxSplitTiles = kCounterBytes / 4;

// Tiles of a shared-ring decode plan as its kernels number them: with M in several row blocks the strips
// are padded to whole groups of eight, so that the row blocks of a strip (tile ids eight apart) share an
// XCD and its L2 holds the strip's B rows once.
int64_t rows_tiles(const dg_gemm_args& a, const TileCfg& t) {
    const int groups = a.gemm_type == kBatched || a.gemm_type == kMasked ? a.num_groups : 1;
    const int64_t nmb = ceil_div(a.m, t.bm), nn = ceil_div(a.n, t.bn);
    return (nmb > 1 ? nmb * align_up64(nn, 8) : nn) * groups;
}

int64_t plan_workspace(const dg_gemm_args& a, const Plan& pl) {
    if (pl.split <= 1) return 0;
    const int64_t tiles = pl.skinny_rows ? rows_tiles(a, pl.tile) : plan_tiles(a, pl.tile);
    return kCounterBytes + tiles * pl.split * (int64_t)pl.tile.bm * pl.tile.bn * 4;
}

// Skinny (M <= 128) dense / batched GEMMs are bound by how many bytes the CUs keep in flight,
// not by MFMA time.  Measured on MI355X (fp8, us): 128x2112x7168 64x128/split 4 17.9 (unsplit
// 27.5), 128x4096x7168 64x128/3 20.6 (unsplit 28.3), 128x7168x16384 128x128/4 40.1,
// 128x7168x2048 64x128/1 13.2 (split 2: 15.5), 128x24576x1536 128x128/1 16.6.  The split
// reduction costs a few microseconds, so K is split only when it is long (about one range per
// 2048 K) and the tiles alone leave CUs idle.
bool skinny_plan(const dg_gemm_args& a, int cus, bool allow_split, Plan& out) {
    if (a.m > 128 || !(a.gemm_type == kNormal || a.gemm_type == kBatched)) return false;
    const TileCfg* t64 = nullptr;
    const TileCfg* t128 = nullptr;
    for (const TileCfg& c : kTiles) {
        if (c.bm == 64 && c.bn == 128) t64 = &c;
        if (c.bm == 128 && c.bn == 128) t128 = &c;
    }
    if (t64 == nullptr || t128 == nullptr) return false;
    const TileCfg& tc = plan_tiles(a, *t64) > cus && a.m > 64 ? *t128 : *t64;
    const int64_t tiles = plan_tiles(a, tc);
    const int ns = ceil_div(a.k, k_stage_elems(a.kind, tc));
    int sp = 1;
    if (allow_split && a.k > 2048 && tiles <= kMaxSplitTiles) {
        sp = (a.k + 1024) / 2048;
        sp = (int)std::min<int64_t>(sp, std::max<int64_t>(1, cus / tiles));
        sp = (int)std::min<int64_t>(sp, std::max<int64_t>(1, (cus / kXcds) / ceil_div64(tiles, kXcds)));
        sp = std::max(1, std::min(sp, 16));
    }
    const int sps = ceil_div(ns, sp);
    out = {tc, ceil_div(ns, sps), sps, 0, 0, 0};
    return true;
}

// DG_GEMV (tuning override), parsed only when its text changes since the last call: "0" = off,
// "ks" or "ks,waves" = forced K split and workgroup size of the GEMV decode kernel; ks = -1 when
// unset.
void gemv_env(int& ks, int& waves) {
    static std::mutex mu;
    static std::string last;
    static int last_ks = -1, last_waves = 0;
    const char* s = std::getenv("DG_GEMV");
    const char* cur = s == nullptr ? "" : s;
    std::lock_guard<std::mutex> lk(mu);
    if (last != cur) {
        last = cur;
        last_ks = -1;
        last_waves = 0;
        if (cur[0] != '\0' && std::sscanf(cur, "%d,%d", &last_ks, &last_waves) < 1) last_ks = -1;
    }
    ks = last_ks;
    waves = last_waves;
}

// DG_SKINNY (tuning override): "0" = never use the skinny-M kernel, "mt,nb,nw,d,ar[,split]" =
// use that configuration wherever M fits it.
struct SkinnyEnv {
    int mode;   // -1 default, 0 off, 1 forced configuration
    int mt, nb, nw, d, ar, split;
    int rows, rmt, rnb, rd, rsplit;   // DG_SKINNY_ROWS: -1 default, 0 off, 1 forced "mt,nb,d[,split[,reduce]]"
    int rreduce;                      // (-1: the plan's choice, 0: last-arriving workgroup, 1: second launch,
                                      //  2: second launch from three K ranges on)
};
SkinnyEnv skinny_env() {
    SkinnyEnv e = {-1, 0, 0, 0, 0, 0, 0, -1, 0, 0, 0, 0, -1};
    const char* rs = std::getenv("DG_SKINNY_ROWS");
    if (rs != nullptr && *rs != '\0') {
        if (std::strcmp(rs, "0") == 0) e.rows = 0;
        else if (std::sscanf(rs, "%d,%d,%d,%d,%d", &e.rmt, &e.rnb, &e.rd, &e.rsplit, &e.rreduce) >= 3) e.rows = 1;
    }
    const char* s = std::getenv("DG_SKINNY");
    if (s == nullptr || *s == '\0') return e;
    if (std::strcmp(s, "0") == 0) { e.mode = 0; return e; }
    if (std::sscanf(s, "%d,%d,%d,%d,%d,%d", &e.mt, &e.nb, &e.nw, &e.d, &e.ar, &e.split) >= 5) e.mode = 1;
    return e;
}

// Decode shapes (dense or batched, M <= 128) stream B through the skinny-M kernel: one
// workgroup per 32-column strip, its four waves splitting K, A staged for the M it holds, and a
// K split across workgroups only while the strips alone leave CUs idle (each range keeps at
// least four 64-K blocks per wave).  Measured on MI355X (fp8, kernel us, tile kernel in
// brackets): M = 1: 2112x7168 8.8 (15.0), 7168x2048 5.7 (13.2), 24576x1536 10.3 (11.5),
// 7168x16384 26.9 (31.7); M = 32: 2112x7168 9.9 (17.1), 7168x2048 6.3 (14.8); M = 64:
// 7168x2048 8.0 (15.9), 4096x7168 14.5 (20.2); M = 128: 7168x2048 11.7 (14.2).  Past 16 rows
// of A, more than two strips per CU (N = 24576) favour the tile kernel (M = 64: 20.1 vs 15.4).
bool skinny_kernel_plan(const dg_gemm_args& a, int cus, bool allow_split, const SkinnyEnv& env, Plan& out) {
    if (env.mode == 0 || !(a.gemm_type == kNormal || a.gemm_type == kBatched || a.gemm_type == kMasked)) return false;
    // (MN-major B is read in place by the skinny kernel's 32-column configurations; MN-major A is not)
    const bool bmn = a.b_mn_major != 0;
    if (a.a_mn_major) return false;
    const int groups0 = a.gemm_type == kNormal ? 1 : a.num_groups;
    // Decode shapes with 64 < M <= 128 (e4m3, bf16, FP8 x FP4; dense or batched; K-major B) take the
    // shared-ring kernel by the rules below: its waves own the tile's 32x32 blocks and fetch each group of
    // B and A once per workgroup, four groups deep.  Measured on MI355X when it was introduced, with 128 x 32
    // strips (fp8, cold L2, event us, skinny kernel in brackets): 128x2112x7168 21.9 (24.8), 128x4096x7168 26.8 (30.0), 128x7168x2048 15.0 (17.0),
    // 96x4096x7168 24.5 (27.6); slower at K = 16384 (87.5 vs 74.5) and for M <= 64 (64x2112x7168
    // 18.6 vs 17.4), which keep the skinny kernel.  The tile shapes below (128 x 64, 64 x 64) replaced
    // the 128 x 32 strips; with them bf16 and FP8 x FP4 (e2m1 B) decode shapes gain too (cold event us,
    // skinny kernel in brackets): FP8 x FP4 128x7168x2048 12.5 (14.0), 128x4096x7168 21.8 (24.4),
    // 128x2112x7168 18.3 (21.4); bf16 128x7168x2048 17.5 (18.5), 128x4096x7168 28.2 (32.6),
    // 128x2112x7168 24.0 (26.2).  (With 128 x 32 strips they had not: bf16 128x4096x7168 29.9 vs 29.0.)
    SkinnyEnv rows_env = env;
    const bool rows_kind = a.kind == kFP8FP8 || a.kind == kFP8FP4 || a.kind == kBF16;
    if (env.rows == -1 && env.mode == -1 && rows_kind && !bmn && a.m > 64 && a.m <= 128 && a.k <= 16384 &&
        (a.gemm_type == kNormal || a.gemm_type == kBatched) && (int64_t)ceil_div(a.n, 32) * groups0 <= 2 * (int64_t)cus) {
        rows_env.rows = 1;
        rows_env.rmt = 4; rows_env.rnb = 1; rows_env.rd = 4; rows_env.rsplit = 0;
        // Long K over many columns: 64-column strips (half the A bytes per column of D), split 2-4 ways
        // to fill the CUs, the partials summed by a second launch (split_reduce_kernel) instead of
        // each strip's last workgroup.  Measured on MI355X (event us, warm, 32-column plan in
        // brackets): 128x4096x7168 20.5 (23.0), 128x3072x7168 19.3 (21.8), 96x4096x7168 19.3 (21.6),
        // 128x6144x7168 26.2 (29.4), 128x7168x7168 27.4 (30.0); level at 128x2112x7168 (18.6 vs
        // 18.7) and behind for K <= 4096 (128x4096x4096 18.9 vs 18.0, 128x7168x4096 21.3 vs 19.7),
        // where the second launch's fixed cost outweighs the saved A traffic.
        const int64_t strips2 = (int64_t)ceil_div(a.n, 64) * groups0;
        // (up to K = 16384, cold event us, skinny kernel in brackets: 128x7168x16384 48.5 (55.8), 128x4096x16384
        // 32.0 (37.4), 128x3072x16384 29.8 (35.7), 128x6144x12288 39.1 (45.8); bf16 128x7168x16384 72.0 (88.8),
        // 128x4096x16384 47.8 (56.4); FP8 x FP4 43.8 (46.7), 29.5 (33.9))
        if (allow_split && a.k > 4096 && a.n >= 3072 && 2 * strips2 <= cus) {
            rows_env.rnb = 2;
            rows_env.rsplit = (int)std::max<int64_t>(2, std::min<int64_t>(4, cus / strips2));
            rows_env.rreduce = 1;
            // From K = 8192 over wide N, 128-column strips (half the A traffic again; cold event us, 64-column
            // plan in brackets): e4m3 128x7168x16384 44.6 (48.4), 96x7168x16384 39.5 (44.2), 128x7168x8192 30.2
            // (31.7), but 128x6144x12288 40.5 (39.4); bf16 128x7168x16384 63.2 (80.6), 128x6144x12288 47.8
            // (59.4), 128x3072x16384 38.0 (43.7), 128x7168x8192 43.8 (45.0), 128x4096x16384 level; FP8 x FP4
            // 128x7168x16384 38.9 (44.0), 96x7168x16384 36.1 (42.5), 128x6144x12288 35.0 (36.2), but
            // 128x4096x16384 30.2 (29.8); below K = 8192 only bf16 over N = 7168 gains (128x7168x7168 38.2
            // (41.4); 128x4096x7168 29.5 (28.6))
            const bool wide128 = a.k >= 8192 ? (a.kind == kBF16 || (a.kind == kFP8FP4 ? a.n >= 6144 : a.n >= 7168))
                                             : a.kind == kBF16 && a.n >= 7168;
            if (wide128) {
                rows_env.rnb = 4;
                rows_env.rsplit = 0;   // (K split to fill the CUs, as measured)
            } else if (a.kind == kFP8FP4 && a.n <= 4096 && a.k <= 8192) {
                // FP8 x FP4 at mid K: 64 x 128 tiles with M in two row blocks, split 4 (cold event us, 128 x 64
                // plan in brackets: 128x4096x7168 20.6 (21.4), 128x3072x7168 19.5 (20.1))
                rows_env.rmt = 2; rows_env.rnb = 4; rows_env.rsplit = 4;
            }
        } else if (allow_split && a.kind == kBF16 && a.k >= 6144 && a.k <= 8192 && a.n >= 2048 && a.n < 3072 &&
                   6 * strips2 <= 2 * (int64_t)cus) {
            // bf16 over about 2112 columns: 128 x 64 tiles split 6 ways, summed by the second launch (cold event
            // us, 64 x 64 plan in brackets: 128x2112x7168 22.6 (23.7), 96x2112x7168 20.6 (23.0))
            rows_env.rnb = 2;
            rows_env.rsplit = 6;
            rows_env.rreduce = 1;
        } else if (a.k > 8192) {
            rows_env.rows = -1;   // (longer K otherwise stays on the skinny kernel)
        } else if (a.m > 80) {
            // Otherwise 64 x 64 tiles (M in two 64-row blocks): at the same number of workgroups each moves
            // ~20 % fewer bytes of A and B than a 128 x 32 strip.  K split as below, the partials summed by
            // the second launch from three ranges on.  Measured on MI355X (event us, cold L2, 128 x 32
            // strips in brackets): 128x2112x7168 19.3 (20.7, split 3), 128x7168x2048 13.4 (14.3),
            // 128x7168x4096 20.0 (21.3), 128x4096x4096 19.2 (20.0), 96x2112x7168 19.1 (20.0); behind
            // where the second block holds few rows (65x4096x1024 13.3 vs 12.5: B read twice for one row).
            rows_env.rmt = 2; rows_env.rnb = 2;
            rows_env.rreduce = 2;   // (second launch when the plan splits K three ways or more)
            // At short K the tiles alone fill the CUs well enough: a two-way split (its last workgroup summing
            // the partials) measured behind the unsplit plan (cold event us, split plan in brackets): e4m3
            // 128x4096x2048 13.1 (16.1), 128x3072x2048 13.0 (15.1), 128x2112x2048 12.8 (14.3), 96x4096x3072
            // 15.9 (16.8); FP8 x FP4 12.2 (15.5), 12.0 (14.6), 12.0 (13.8), 128x4096x4096 17.3 (18.2); bf16
            // 128x4096x2048 16.4 (17.7), 128x3072x2048 16.3 (16.8), but 128x2112x2048 16.0 (15.0), and
            // 128x2112x4096 splits better for every kind (e4m3 16.0 vs 18.7)
            const bool short_k = a.kind == kBF16 ? a.k <= 2048 && a.n >= 3072
                                                 : (a.k <= 3072 && a.n >= 2048) || (a.kind == kFP8FP4 && a.k <= 4096 && a.n >= 4096);
            if (short_k) rows_env.rsplit = 1;
            // bf16 rows of 8 KB and more in an unsplit plan stay on the skinny kernel (128x7168x4096
            // 37.1 vs 29.1 us; split or shorter rows gain: 128x4096x4096 23.2 vs 24.2, 128x7168x3072
            // 23.0 vs 24.9, 128x2112x7168 24.0 vs 26.2)
            const int64_t tiles64 = (int64_t)ceil_div(a.n, 64) * 2 * groups0;
            const bool unsplit = !allow_split || cus / tiles64 <= 1 || ceil_div(a.k, 64) < 16;
            if (a.kind == kBF16 && unsplit && a.k >= 4096) rows_env.rows = -1;
        } else if (a.kind != kFP8FP8) {
            rows_env.rows = -1;   // (128 x 32 strips measured no gain over the skinny kernel for these kinds)
        }
    }
    // e4m3 with 32 < M <= 64 and long K over many columns: 64 x 128 tiles, split-K partials summed by the
    // second launch (cold event us, skinny kernel in brackets, two boxes: 64x7168x16384 35.1 (38.6) and 39.4
    // (40.7), 64x4096x16384 25.5 (26.8) and 25.5 (27.2); at K = 7168 it measured level or behind: 64x4096x7168
    // 19.1 (18.6), 64x7168x7168 22.8 (21.8))
    // bf16 rows (twice the bytes per K) gain from K > 4096: 64 x 128 tiles from N >= 6144, 64 x 64 below
    // (cold event us, skinny kernel in brackets: 64x7168x16384 51.6 (61.3), 64x7168x7168 30.5 (33.5),
    // 64x4096x7168 21.9 (23.9), 64x4096x16384 42.6 (43.0); 64x2112x7168 22.1 (19.2) keeps the skinny kernel)
    const bool m64_rows = env.rows == -1 && env.mode == -1 && !bmn && a.m > 32 && a.m <= 64 && a.k <= 16384 &&
                          allow_split && (a.gemm_type == kNormal || a.gemm_type == kBatched);
    if (m64_rows && a.kind == kFP8FP8 && a.k > 8192 && a.n >= 4096 && (int64_t)ceil_div(a.n, 128) * groups0 <= (int64_t)cus) {
        rows_env.rows = 1;
        rows_env.rmt = 2; rows_env.rnb = 4; rows_env.rd = 4; rows_env.rsplit = 0; rows_env.rreduce = 1;
    } else if (m64_rows && a.kind == kBF16 && a.k > 4096 && a.n >= 3072 &&
               (int64_t)ceil_div(a.n, 64) * groups0 <= (int64_t)cus) {
        rows_env.rows = 1;
        rows_env.rmt = 2; rows_env.rnb = a.n >= 6144 ? 4 : 2; rows_env.rd = 4; rows_env.rsplit = 0; rows_env.rreduce = 1;
    }
    // (dense and batched launches may hold M in several tiles of 32 mt rows, M <= 128)
    const bool rows_mblocks = (a.gemm_type == kNormal || a.gemm_type == kBatched) && a.m <= 128;
    if (rows_env.rows == 1 && !bmn && (a.m <= 32 * rows_env.rmt || rows_mblocks) &&
        lookup_skinny_rows(a.kind, rows_env.rmt, rows_env.rnb, rows_env.rd, kEpiBf16) != nullptr) {
        const SkinnyEnv& env = rows_env;
        // shared-ring decode kernel: K split across workgroups while the tiles leave CUs idle,
        // each range keeping at least eight 64-K blocks
        const int64_t strips = (int64_t)ceil_div(a.n, 32 * env.rnb) * ceil_div(a.m, 32 * env.rmt) * groups0;
        const int nk64 = std::max(1, ceil_div(a.k, 64));
        int sp = 1;
        if (allow_split && strips <= kMaxSplitTiles) {
            sp = env.rsplit > 0 ? env.rsplit : (int)std::min<int64_t>(std::max<int64_t>(1, cus / strips), std::max(1, nk64 / 8));
            sp = std::max(1, std::min(sp, std::min(16, nk64)));
        }
        const int ss = ceil_div(nk64, sp);
        out = {{32 * env.rmt, 32 * env.rnb, 0, env.rmt * env.rnb, 0, 0, 0, 0, 0}, ceil_div(nk64, ss), ss,
               env.rmt * env.rnb, env.rd, 32 * env.rmt, 1, 0, 0};
        out.split_reduce = (out.split > 1 && env.rreduce == 1) || (out.split > 2 && env.rreduce == 2) ? 1 : 0;
        return true;
    }
    int mt = a.m <= 32 ? 1 : (a.m <= 64 ? 2 : 4), nb = 1, nw = 4, d = 2, ar = a.m <= 16 ? 16 : 32 * mt;
    // long K over at most one strip per CU: eight waves per strip keep more of it in flight
    // (M = 1, 7168x16384: 24.4 vs 26.9 us; bf16 rows, twice the bytes per K, keep four waves:
    // 46.6 vs 50.3 us cold)
    if (a.m <= 16 && a.k >= 8192 && a.kind != kBF16 && (int64_t)ceil_div(a.n, 32) * groups0 <= cus)
        nw = 8;
    if (env.mode == 1) {
        mt = env.mt; nb = env.nb; nw = env.nw; d = env.d; ar = env.ar;
    } else if (a.m > 128 || (a.m > 16 && !bmn && (int64_t)ceil_div(a.n, 32) * groups0 > 2 * (int64_t)cus)) {
        // (MN-major B keeps the skinny kernel over many strips: the tile plans would copy B first)
        return false;
    }
    if (a.m > ar || (bmn ? lookup_skinny_mn(a.kind, mt, nb, nw, d, ar, kEpiBf16)
                         : lookup_skinny(a.kind, mt, nb, nw, d, ar, kEpiBf16)) == nullptr)
        return false;
    const int64_t strips = (int64_t)ceil_div(a.n, 32 * nb) * groups0;
    const int nk64 = std::max(1, ceil_div(a.k, 64));
    int sp = 1;
    if (allow_split && strips <= kMaxSplitTiles) {
        if (env.mode == 1 && env.split > 0) sp = env.split;
        else sp = (int)std::min<int64_t>(std::max<int64_t>(1, cus / strips), std::max(1, nk64 / (4 * nw)));
        // (K <= 2048 stays unsplit, e4m3 up to K = 3072: cold event us, split 2 in brackets: e4m3 64x4096x2048
        // 10.9 (12.8), 64x3072x2048 10.8 (12.3), 64x2112x2048 10.6 (11.9), 32x4096x2048 10.2 (10.8),
        // 16x4096x2048 9.0 (10.3), 1x4096x2048 8.6 (10.3), 1x3072x3072 9.7 (10.9), 16x2112x3072 10.0 (10.5);
        // bf16 64x4096x2048 13.4 (14.2), 16x4096x2048 10.6 (11.3), 1x4096x2048 10.3 (11.2), 64x2112x2048 13.1
        // (12.8), but 16x2112x3072 12.7 (11.4))
        if (env.mode != 1 && (nk64 <= 32 || (a.kind == kFP8FP8 && nk64 <= 48))) sp = 1;
        sp = std::max(1, std::min(sp, std::min(16, nk64)));
    }
    const int ss = ceil_div(nk64, sp);
    out = {{32 * mt, 32 * nb, 0, nw, 0, 0, 0, 0, 0}, ceil_div(nk64, ss), ss, nw, d, ar};
    return true;
}

// Tiles with a persistent kernel (csrc/gemm_persistent.hpp): the 128-K-stage tiles whose
// persistent body fits the register file (256x256 does not).
bool tile_persistable(const TileCfg& t) {
    return t.km == 2 && t.stages == 2 && !(t.bm == 256 && t.bn == 256) && !tile_anchored(t.bm);
}

// CUs the launch may occupy are capped below the device's (set_num_sms).
bool cus_capped(int cus) { return cus < device_cus(); }

Plan select_plan(const dg_gemm_args& a, int cus, bool allow_split) {
    Plan skinny;
    if (skinny_kernel_plan(a, cus, allow_split, skinny_env(), skinny)) return skinny;
    if (skinny_plan(a, cus, allow_split, skinny)) return skinny;
    // M-grouped layouts whose alignment rules out 256-row tiles take 384x192 tiles anchored at each
    // group's (m_indices: each run's) first row: a group of up to 384 rows streams its weights once instead of once
    // per 128-row block.  Measured (G = 32 routed top-8 counts, ~257 rows a group, alignment 128,
    // cold us): N=4096 K=7168 345.6 vs 458.7 (128x256), N=7168 K=2048 200.3 vs 237.9; bf16
    // 635.6 vs 839.9 and 330.2 vs 408.5.  With alignment 256 the 256-row tiles are faster (443 vs
    // 526 at N=4096 K=7168).
    // (e2m1 B takes 384x128: its 384x192 build spills 148-192 bytes per lane and ran 2.5x behind, G=32 routed,
    // alignment 128, cold us: N=4096 K=7168 1011 vs 370 on 384x128 and 410 on the scored 128x256, N=7168
    // K=2048 532 vs 217 / 219)
    const bool fp4_b = a.kind == kFP8FP4 || a.kind == kFP4FP4;
    if ((a.gemm_type == kMGroupedPsum || a.gemm_type == kMGroupedIdx) && a.alignment % 256 != 0) {
        for (const TileCfg& tc : kTiles)
            if (tc.bm == 384 && tc.bn == (fp4_b ? 128 : 192)) return {tc, 1, ceil_div(a.k, k_stage_elems(a.kind, tc)), 0, 0, 0};
    }
    allow_split = false;   // wide problems fill the CUs with tiles
    const int groups = (a.gemm_type == kBatched || a.gemm_type == kMasked || a.gemm_type == kKGrouped) ? a.num_groups : 1;
    // (K-grouped: each tile contracts one group's share of K)
    const int k_tile = a.gemm_type == kKGrouped ? ceil_div(a.k, std::max(1, a.num_groups)) : a.k;
    // HBM floor: operands once, D once (8 TB/s at ~2.1 GHz is ~3800 bytes per cycle).
    const double esz = a.kind == kBF16 ? 2.0 : 1.0;
    // (The plan must not depend on D's dtype: a bf16 D is then exactly the RNE rounding of the
    // fp32 D of the same call, with the same K split and summation order.)
    const double hbm_bytes = esz * ((double)a.m + a.n) * a.k * groups + 2.0 * a.m * a.n * groups;
    double best = 1e300;
    Plan pick = {{0, 0, 0, 0, 0, 0, 0, 0, 0}, 1, 1, 0, 0, 0};
    for (int i = 0; i < kNumTiles; ++i) {
        const TileCfg& tc = kTiles[i];
        // (anchored tiles only where the alignment rules out 256-row tiles, above: at alignment 256 they
        // measured behind, 526 vs 443 us for 256x224 at G=32 N=4096 K=7168, and FP8 x FP4 G=8 x 4096
        // rows N=7168 K=3072 took 2546 us on 384x192)
        if (!tile_allowed(a, tc.bm, tc.bn) || tile_anchored(tc.bm)) continue;
        const int ns = ceil_div(k_tile, k_stage_elems(a.kind, tc));
        const int64_t tiles = plan_tiles(a, tc);
        const int max_split = allow_split && tile_splittable(tc) && tiles <= kMaxSplitTiles ? std::min(16, std::max(1, ns / 4)) : 1;
        for (int sp = 1; sp <= max_split; ++sp) {
            const int sps = ceil_div(ns, sp);
            const int s_eff = ceil_div(ns, sps);
            if (sp > 1 && s_eff != sp) continue;
            // The splits of a tile run on one XCD (kXcds of them, cus / kXcds CUs each).
            const int64_t rounds = sp == 1 ? ceil_div64(tiles, (int64_t)cus * tc.occ)
                                           : ceil_div64(ceil_div64(tiles, kXcds) * sp, std::max(1, cus / kXcds));
            if (sp > 1 && rounds > 1) break;
            // Waves of workgroups x (their K stages at the tile's measured stage time + the
            // fixed cost of a tile: pipeline fill and the epilogue's stores), plus the split
            // reduction (measured ~10K cycles: partial stores, arrival count, partial reads).
            // (co-resident workgroups share the CU's MFMAs but overlap each other's fixed costs)
            double t = (double)rounds * ((double)tc.occ * sps * tc.km * tc.stage_cycles + 6000.0 + tc.bm * tc.bn / 8.0);
            double bytes = hbm_bytes;
            if (sp > 1) {
                t += 10000.0 + 500.0 * sp;
                bytes += 8.0 * a.m * a.n * groups * sp;
            }
            t = std::max(t, bytes / 3800.0);
            if (t < best * 0.97) {
                best = t;
                pick = {tc, sp, sps, 0, 0, 0};
            }
        }
    }
    return pick;
}

struct MemoKey {
    int kind, type, m, n, k, g, cus, align, allow_split, mn;
    SkinnyEnv skinny;
    bool operator==(const MemoKey& o) const { return memcmp(this, &o, sizeof(*this)) == 0; }
};
struct MemoHash {
    size_t operator()(const MemoKey& k) const {
        size_t h = 1469598103934665603ull;
        const unsigned char* p = reinterpret_cast<const unsigned char*>(&k);
        for (size_t i = 0; i < sizeof(k); ++i) h = (h ^ p[i]) * 1099511628211ull;
        return h;
    }
};

std::mutex g_memo_mu;
std::unordered_map<MemoKey, Plan, MemoHash> g_memo;

Plan choose(const dg_gemm_args& a, int cus, bool allow_split) {
    allow_split = allow_split && split_capable(a);
    if (a.block_m > 0 && a.block_n > 0) {
        TileCfg t = {a.block_m, a.block_n, 0, 0, 0, 0, 0, 0, 0};
        for (const TileCfg& c : kTiles)
            if (c.bm == a.block_m && c.bn == a.block_n) t = c;
        const int ns = ceil_div(a.k, k_stage_elems(a.kind, t));
        int sp = allow_split && tile_splittable(t) && a.split_k > 1 && plan_tiles(a, t) <= kMaxSplitTiles ? std::min(a.split_k, std::max(1, ns)) : 1;
        const int sps = ceil_div(ns, sp);
        return {t, ceil_div(ns, sps), sps, 0, 0, 0};
    }
    MemoKey key;
    memset(&key, 0, sizeof(key));
    key.kind = a.kind; key.type = a.gemm_type; key.m = a.m; key.n = a.n; key.k = a.k;
    key.g = a.num_groups; key.cus = cus; key.align = a.alignment;
    key.allow_split = allow_split && a.split_k != 1;
    key.mn = (a.a_mn_major ? 1 : 0) | (a.b_mn_major ? 2 : 0);
    key.skinny = skinny_env();
    Plan pl;
    {
        std::lock_guard<std::mutex> lk(g_memo_mu);
        auto it = g_memo.find(key);
        if (it != g_memo.end()) {
            pl = it->second;
        } else {
            pl = select_plan(a, cus, key.allow_split);
            g_memo.emplace(key, pl);
        }
    }
    if (pl.skinny_nw > 0) {
        if (allow_split && a.split_k > 1 && plan_tiles(a, pl.tile) <= kMaxSplitTiles) {
            // forced split count (tuning), in 64-K blocks
            const int nk64 = std::max(1, ceil_div(a.k, 64));
            const int ss = ceil_div(nk64, std::min(a.split_k, nk64));
            pl.split = ceil_div(nk64, ss);
            pl.split_stages = ss;
        }
        return pl;
    }
    if (allow_split && tile_splittable(pl.tile) && a.split_k > 1 && plan_tiles(a, pl.tile) <= kMaxSplitTiles) {
        // forced split count (tuning), on the heuristic's tile shape
        const int ns = ceil_div(a.k, k_stage_elems(a.kind, pl.tile));
        const int sps = ceil_div(ns, std::min(a.split_k, std::max(1, ns)));
        pl.split = ceil_div(ns, sps);
        pl.split_stages = sps;
    }
    return pl;
}

int elem_bytes_times2(int kind, bool is_a) {
    // storage bytes per 2 logical K elements
    switch (kind) {
        case kFP8FP8: return 2;
        case kFP8FP4: return is_a ? 2 : 1;
        case kFP4FP4: return 1;
        case kBF16: return 4;
    }
    return 0;
}

}  // namespace dg

extern "C" int dg_select_config(const dg_gemm_args* args, int32_t* block_m, int32_t* block_n) {
    if (args == nullptr) return dg_set_error("dg_select_config: null args");
    const int cus = args->num_cus > 0 ? args->num_cus : dg::device_cus();
    const dg::Plan pl = dg::choose(*args, cus, args->workspace != nullptr || args->library_workspace != 0 || args->split_k > 1);
    if (pl.tile.bm == 0) return dg_set_error("no tile shape fits this problem (M-grouped alignment must be a multiple of 32)");
    if (block_m) *block_m = pl.tile.bm;
    if (block_n) *block_n = pl.tile.bn;
    return DG_OK;
}

extern "C" int dg_gemm_workspace_size(const dg_gemm_args* args, int64_t* bytes) {
    if (args == nullptr || bytes == nullptr) return dg_set_error("dg_gemm_workspace_size: null argument");
    *bytes = 0;
    if (args->m <= 0 || args->n <= 0 || args->k <= 0) return DG_OK;
    const int cus = args->num_cus > 0 ? args->num_cus : dg::device_cus();
    const dg::Plan pl = dg::choose(*args, cus, true);
    if (pl.tile.bm == 0) return dg_set_error("no tile shape fits this problem (M-grouped alignment must be a multiple of 32)");
    *bytes = dg::plan_workspace(*args, pl);
    return DG_OK;
}

namespace {

// Launches an ahead-of-time kernel through hipModuleLaunchKernel: its hipFunction_t handle is
// looked up once (hipGetFuncBySymbol) and cached per kernel.
std::mutex g_func_mu;
std::unordered_map<const void*, hipFunction_t> g_funcs;

hipError_t launch_module_kernel(const void* kernel, unsigned grid, unsigned threads, dg::KParams& p, hipStream_t st,
                                unsigned lds_bytes = 0) {
    hipFunction_t f = nullptr;
    {
        std::lock_guard<std::mutex> lk(g_func_mu);
        auto it = g_funcs.find(kernel);
        if (it != g_funcs.end()) {
            f = it->second;
        } else {
            const hipError_t e = hipGetFuncBySymbol(&f, kernel);
            if (e != hipSuccess) return e;
            g_funcs.emplace(kernel, f);
        }
    }
    void* params[] = {&p};
    return hipModuleLaunchKernel(f, grid, 1, 1, threads, 1, 1, lds_bytes, st, params, nullptr);
}

// Split-K workspaces the library owns, one per (device, stream): zero-filled when allocated, left
// zero-filled by every launch (so calls issued in order on one stream share one), only ever grown,
// and never freed -- a graph captured on the stream may still hold an older one.  Calls that run
// at the same time on one stream's workspace (a graph replayed on another stream while the capture
// stream runs eager calls) race on its counters.
struct StreamWorkspace {
    void* ptr = nullptr;
    int64_t bytes = 0;
};
std::mutex g_stream_ws_mu;
// Slot 0 holds the split-K workspace, slot 1 the run table of an anchored m_indices GEMM.
std::map<std::tuple<int, hipStream_t, int>, StreamWorkspace> g_stream_ws;

int stream_workspace(hipStream_t st, int64_t need, void** out, int slot = 0) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return dg_set_error("dg_gemm: no current HIP device");
    std::lock_guard<std::mutex> lk(g_stream_ws_mu);
    StreamWorkspace& w = g_stream_ws[{dev, st, slot}];
    if (w.bytes >= need) {
        *out = w.ptr;
        return DG_OK;
    }
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(st, &cs) != hipSuccess) (void)hipGetLastError();
    if (cs != hipStreamCaptureStatusNone) {
        char buf[256];
        snprintf(buf, sizeof(buf), "dg_gemm: this call needs a %lld-byte workspace but the stream's is %lld "
                 "bytes, and it cannot grow while the stream is being captured: run the same call once before "
                 "the capture", (long long)need, (long long)w.bytes);
        return dg_set_error(buf);
    }
    const int64_t bytes = std::max<int64_t>({need, 2 * w.bytes, int64_t(1) << 20});
    void* p = nullptr;
    hipError_t e = hipMalloc(&p, (size_t)bytes);
    if (e == hipSuccess) e = hipMemsetAsync(p, 0, (size_t)bytes, st);   // (never inside a capture: checked above)
    if (e != hipSuccess) {
        std::string msg = std::string("dg_gemm: workspace allocation failed: ") + hipGetErrorString(e);
        return dg_set_error(msg.c_str());
    }
    w.ptr = p;
    w.bytes = bytes;
    *out = p;
    return DG_OK;
}

// Checks, plans and launches one GEMM; with `info` it stops short of the launch and describes it.
int gemm_impl(const dg_gemm_args* args, void* stream, bool compile_only, dg_launch_info* info = nullptr,
              bool noalloc = false) {
    using namespace dg;
    if (args == nullptr) return dg_set_error("dg_gemm: null args");
    const dg_gemm_args& a = *args;
    if (a.kind < kFP8FP8 || a.kind > kBF16) return dg_set_error("dg_gemm: unknown kind");
    if (a.gemm_type < kNormal || a.gemm_type > kKGrouped) return dg_set_error("dg_gemm: unknown gemm_type");
    if (a.m < 0 || a.n < 0 || a.k < 0) return dg_set_error("dg_gemm: negative size");
    if (a.d_dtype != DG_DTYPE_BF16 && a.d_dtype != DG_DTYPE_F32 && a.d_dtype != DG_DTYPE_FP8_E4M3)
        return dg_set_error("dg_gemm: D must be bf16, fp32 or e4m3");
    if (a.epilogue != DG_EPI_DEFAULT && a.epilogue != DG_EPI_BF16_SR) return dg_set_error("dg_gemm: unknown epilogue");
    if (a.epilogue == DG_EPI_BF16_SR &&
        (a.d_dtype != DG_DTYPE_BF16 || a.accumulate || a.bias != nullptr || a.alpha != 1.0f))
        return dg_set_error("Stochastic rounding requires a direct BF16 output");
    if (a.d_dtype == DG_DTYPE_FP8_E4M3) {
        if (a.kind != kFP8FP8 || (a.gemm_type != kNormal && a.gemm_type != kBatched))
            return dg_set_error("dg_gemm: FP8 output needs e4m3 operands and a dense or batched GEMM");
        if (a.accumulate || a.bias != nullptr || a.alpha != 1.0f || a.epilogue != DG_EPI_DEFAULT)
            return dg_set_error("FP8 quantization requires a direct E4M3 output");
        if (a.n % 128 != 0) return dg_set_error("FP8 output requires N to be a multiple of 128");
        if (a.sfd == nullptr || a.sfd_ld < a.m) return dg_set_error("dg_gemm: FP8 output needs sfd with sfd_ld >= m");
        if (a.ldd % 4 || (reinterpret_cast<uintptr_t>(a.d) & 3) || (a.gemm_type == kBatched && a.batch_stride_d % 4))
            return dg_set_error("dg_gemm: FP8 output rows must be 4-byte aligned");
    }
    if (info != nullptr) memset(info, 0, sizeof(*info));
    if (a.m == 0 || a.n == 0) return DG_OK;
    const bool bf16 = a.kind == kBF16;
    // (a launch-plan query needs sizes and strides only)
    const bool plan_only = info != nullptr;
    if (!plan_only && (a.a == nullptr || a.b == nullptr || a.d == nullptr)) return dg_set_error("dg_gemm: null operand");
    if (!plan_only && !bf16 && (a.sfa == nullptr || a.sfb == nullptr)) return dg_set_error("dg_gemm: scale factors required");
    const bool grouped = a.gemm_type != kNormal;
    if (!plan_only && (a.gemm_type == kMGroupedPsum || a.gemm_type == kMGroupedIdx || a.gemm_type == kMasked ||
                       a.gemm_type == kKGrouped) &&
        a.grouped_layout == nullptr)
        return dg_set_error("dg_gemm: grouped_layout required");
    if (grouped && a.num_groups < 1) return dg_set_error("dg_gemm: num_groups must be >= 1");
    if (grouped && a.accumulate && a.gemm_type != kBatched && a.gemm_type != kKGrouped)
        return dg_set_error("dg_gemm: grouped GEMMs do not accumulate");
    if (a.gemm_type == kKGrouped && (a.alignment < 64 || a.alignment % 64 != 0))
        return dg_set_error("dg_gemm: K-grouped alignment must be a multiple of 64");
    // storage bytes of one K row
    const int64_t kbytes_a = (int64_t)a.k * elem_bytes_times2(a.kind, true) / 2;
    const int64_t kbytes_b = (int64_t)a.k * elem_bytes_times2(a.kind, false) / 2;
    const int64_t esz_a = bf16 ? 2 : 1, esz_b = bf16 ? 2 : 1;
    const int64_t lda_b = a.lda * esz_a, ldb_b = a.ldb * esz_b;
    if ((a.kind == kFP4FP4 && a.k % 2) || (a.kind == kFP8FP4 && a.k % 2))
        return dg_set_error("dg_gemm: packed FP4 operands need an even K");
    if (kbytes_a % 16 || kbytes_b % 16 || lda_b % 16 || ldb_b % 16 ||
        (reinterpret_cast<uintptr_t>(a.a) & 15) || (reinterpret_cast<uintptr_t>(a.b) & 15))
        return dg_set_error("dg_gemm: K rows and strides must be 16-byte aligned (host pads otherwise)");
    // MN-major operands ([K][MN] storage, read in place by the 128-K-stage tile kernels)
    const bool amn = a.a_mn_major != 0, bmn = a.b_mn_major != 0;
    const bool mgrouped = a.gemm_type == kMGroupedPsum || a.gemm_type == kMGroupedIdx;
    if ((amn || bmn) && ((a.kind != kFP8FP8 && a.kind != kBF16) || a.jit || (mgrouped && amn) ||
                         !(a.gemm_type == kNormal || a.gemm_type == kBatched || a.gemm_type == kKGrouped || mgrouped))) {
        dg_set_error("dg_gemm: MN-major operands are read in place only by e4m3 / bf16 dense, batched and "
                     "K-grouped ahead-of-time kernels (M-grouped: B only)");
        return DG_ENOKERNEL;
    }
    if ((amn ? lda_b < a.m * esz_a : lda_b < kbytes_a) || (bmn ? ldb_b < a.n * esz_b : ldb_b < kbytes_b) || a.ldd < a.n)
        return dg_set_error("dg_gemm: leading dimension smaller than the row");
    // (an MN-major operand's whole K extent must fit a buffer range below the dead-load offset)
    if ((amn ? (int64_t)a.k * lda_b >= 0x40000000LL : (int64_t)256 * lda_b > 0x7fffffffLL) ||
        (bmn ? (int64_t)a.k * ldb_b >= 0x40000000LL : (int64_t)256 * ldb_b > 0x7fffffffLL))
        return dg_set_error("dg_gemm: row stride too large for 32-bit tile offsets");
    if (!bf16 && ((a.sfa_ld | a.sfb_ld | a.sfa_batch_stride | a.sfb_batch_stride) & 1))
        return dg_set_error("dg_gemm: SF leading dimensions and batch strides must be even (int16 elements)");
    if (a.gemm_type == kMGroupedPsum || a.gemm_type == kMGroupedIdx) {
        if (a.alignment < 32 || a.alignment % 32 != 0) return dg_set_error("dg_gemm: alignment must be a multiple of 32");
    }

    const int cus = a.num_cus > 0 ? a.num_cus : device_cus();
    if (a.split_k < 0) return dg_set_error("dg_gemm: split_k must be >= 0");
    const bool lib_ws = a.workspace == nullptr && a.library_workspace != 0;
    Plan plan = choose(a, cus, a.workspace != nullptr || lib_ws);
    void* workspace = a.workspace;
    if (plan.split > 1 && lib_ws) {
        if (!plan_only && !compile_only) {
            const int rc = stream_workspace(reinterpret_cast<hipStream_t>(stream), plan_workspace(a, plan), &workspace);
            if (rc != DG_OK) return rc;
        }
    } else if (plan.split > 1 && plan_workspace(a, plan) > a.workspace_bytes) {
        if (a.split_k > 1) return dg_set_error("dg_gemm: workspace smaller than dg_gemm_workspace_size() reports");
        plan = choose(a, cus, false);
    }
    const TileCfg cfg = plan.tile;
    if (cfg.bm == 0) return dg_set_error("dg_gemm: no tile shape fits this problem");
    // (MN-major B also in the skinny kernel's 32-column plans)
    const bool skinny_mn = bmn && !amn && plan.skinny_nw > 0 && !plan.skinny_rows && cfg.bn == 32;
    if ((amn || bmn) && !skinny_mn && (plan.skinny_nw > 0 || plan.split != 1 || cfg.km != 2 || cfg.stages != 2 ||
                                       cfg.bm > 256 || cfg.bn > 256)) {
        dg_set_error("dg_gemm: MN-major operands need a 128-byte-stage tile plan (large M and N); this problem "
                     "plans another kernel");
        return DG_ENOKERNEL;
    }
    if (!tile_allowed(a, cfg.bm, cfg.bn)) return dg_set_error("dg_gemm: block_m must divide the M-grouped alignment");
    // Direct register stores measured faster than staging the tile through LDS.
    const int epi_kind = a.d_dtype == DG_DTYPE_F32 ? kEpiF32
                       : a.d_dtype == DG_DTYPE_FP8_E4M3 ? kEpiFp8
                       : a.epilogue == DG_EPI_BF16_SR ? kEpiBf16SR : kEpiBf16;
    // Decode GEMV kernel (e4m3 x e4m3, dense or batched, fp32 / bf16 D without an output
    // epilogue): workgroups of 8 waves over groups of 8 rows of B, K split ks ways between the
    // waves of a workgroup (never across workgroups); ks doubles (up to 8) while each K range keeps
    // at least 8 steps of 128 bytes.  By default for M = 1 with 4096 <= K <= 8192, where it measured
    // ahead of the MFMA decode kernel (MI355X, kernel us, cold L2, two boxes: 1x2112x7168 7.3 vs
    // 9.0-9.3, 1x4096x7168 8.8-8.9 vs 10.4-10.5); level at 1x7168x16384 (24.2-24.4 vs 23.0-25.4),
    // behind at 1x7168x2048 (6.1 vs 5.8), 1x24576x1536 (11.1 vs 10.4) and for M = 2 (2x2112x7168
    // 9.5 vs 8.8), where the VALU work per byte of B doubles.  DG_GEMV forces it for M <= 4 (with ks = 1, 2,
    // 4 or 8, optionally ",4" for four-wave workgroups; "0" turns it off).  Not
    // under a forced plan (tuning overrides).
    int gemv_mr = 0, gemv_ks = 0, gemv_waves = 0;
    {
        // DG_GEMV (tuning): "0" = off, "ks" or "ks,waves" = forced K split (1, 2, 4, 8) and workgroup size (4, 8)
        int env_ks = -1, env_waves = 0;
        gemv_env(env_ks, env_waves);
        const int mr = a.m <= 1 ? 1 : a.m <= 2 ? 2 : 4;
        const bool wanted = env_ks > 0 ? a.m <= 4 : env_ks == -1 && a.m == 1 && a.k >= 4096 && a.k <= 8192;
        if (wanted && a.kind == kFP8FP8 && (a.gemm_type == kNormal || a.gemm_type == kBatched) && a.m >= 1 &&
            a.k > 0 && !amn && !bmn && (epi_kind == kEpiF32 || epi_kind == kEpiBf16) && a.block_m <= 0 &&
            a.split_k <= 1 && skinny_env().mode == -1) {
            const int pk = ceil_div(a.k, 128);
            int ks = 1;
            if (env_ks == 1 || env_ks == 2 || env_ks == 4 || env_ks == 8) ks = env_ks;
            else {
                // (and while the workgroups of 8 waves still fit one round on the CUs: 1x7168x4096 11.7 vs
                // 13.4 us at ks 2 / 4, 1x7168x7168 16.1 vs 16.9; cold event us)
                const int64_t gb = a.gemm_type == kBatched ? a.num_groups : 1;
                while (ks < 8 && pk >= 16 * ks && (int64_t)ceil_div(a.n, 32 / ks) * gb <= cus) ks *= 2;
            }
            // eight-wave workgroups (two waves per SIMD); four-wave ones (half the rows each, twice the
            // workgroups) measured slower even where eight-wave ones leave CUs idle (1x2112x7168,
            // ks 4: 7.8 vs 7.2 us on 264 vs 132 CUs), so they are a tuning option only
            int waves = env_waves == 4 || env_waves == 8 ? env_waves : 8;
            if (ks > waves) waves = 8;
            if (gemv_lds(mr, a.k, ks) <= 64 * 1024 && 64LL * ldb_b < 0x40000000LL &&
                (int64_t)ceil_div(a.k, 64) * a.sfb_ld * 2 + 2 * (int64_t)a.n < 0x7fffffffLL &&
                lookup_gemv(mr, epi_kind, waves) != nullptr) {
                gemv_mr = mr;
                gemv_ks = ks;
                gemv_waves = waves;
            }
        }
    }
    // (the skinny-M kernel is not specialised per problem: the JIT setting leaves it ahead-of-time)
    const bool skinny = plan.skinny_nw > 0 || gemv_mr > 0;
    const bool jit = a.jit && !skinny;
    if (skinny && compile_only && info == nullptr) return DG_OK;
    // Persistent launch (one workgroup per CU walking the tiles, the LDS ring running on across
    // them): the 128-K-stage tiles of unsplit GEMMs whose operand tensors fit 31-bit offsets.
    const int groups_all = (a.gemm_type == kBatched || a.gemm_type == kMasked) ? a.num_groups : 1;
    const int groups_b = a.gemm_type == kNormal ? 1 : a.num_groups;
    const int64_t nk64 = ceil_div(a.k, 64);
    const int64_t a_span = (int64_t)(groups_all - 1) * a.batch_stride_a * esz_a + (int64_t)(a.m - 1) * lda_b + kbytes_a;
    const int64_t b_span = (int64_t)(groups_b - 1) * a.batch_stride_b * esz_b + (int64_t)(a.n - 1) * ldb_b + kbytes_b;
    const int64_t sfa_span = bf16 ? 0 : ((int64_t)(groups_all - 1) * a.sfa_batch_stride + nk64 * a.sfa_ld) * 2;
    const int64_t sfb_span = bf16 ? 0 : ((int64_t)(groups_b - 1) * a.sfb_batch_stride + nk64 * a.sfb_ld) * 2;
    // The persistent kernel runs where the launch must stay within `cus` CUs (set_num_sms below the
    // device's count) or when DG_PERSISTENT=1 asks for it (tuning); it measured no faster than
    // one tile per workgroup at full occupancy (the same ring, the epilogue still not overlapped).
    static const char* persist_env = std::getenv("DG_PERSISTENT");
    const bool want_persistent = cus_capped(cus) || (persist_env != nullptr && persist_env[0] == '1');
    const bool persistent = want_persistent && !jit && !skinny && !amn && !bmn && plan.split == 1 && tile_persistable(cfg) &&
                            a.k > 0 && a.gemm_type != kKGrouped && a_span <= 0x7fffffffLL &&
                            b_span <= 0x7fffffffLL && sfa_span <= 0x7fffffffLL && sfb_span <= 0x7fffffffLL;
    KernelFn fn = jit ? nullptr
                : skinny ? (plan.skinny_rows ? lookup_skinny_rows(a.kind, cfg.bm / 32, cfg.bn / 32, plan.skinny_d, epi_kind)
                          : skinny_mn ? lookup_skinny_mn(a.kind, cfg.bm / 32, cfg.bn / 32, plan.skinny_nw, plan.skinny_d, plan.skinny_ar, epi_kind)
                                      : lookup_skinny(a.kind, cfg.bm / 32, cfg.bn / 32, plan.skinny_nw, plan.skinny_d, plan.skinny_ar, epi_kind))
                : (amn || bmn) ? lookup_kernel_mn(a.kind, cfg.bm, cfg.bn, epi_kind, amn, bmn)
                         : lookup_kernel(a.kind, cfg.bm, cfg.bn, epi_kind, persistent);
    if (fn == nullptr && !jit) {
        char buf[160];
        snprintf(buf, sizeof(buf), "dg_gemm: no compiled kernel for kind=%d block=%dx%d", a.kind, cfg.bm, cfg.bn);
        dg_set_error(buf);
        return DG_ENOKERNEL;
    }

    KParams p;
    memset(&p, 0, sizeof(p));
    p.a = reinterpret_cast<const uint8_t*>(a.a);
    p.b = reinterpret_cast<const uint8_t*>(a.b);
    p.d = reinterpret_cast<uint8_t*>(a.d);
    p.sfa = reinterpret_cast<const uint16_t*>(a.sfa);
    p.sfb = reinterpret_cast<const uint16_t*>(a.sfb);
    p.bias = reinterpret_cast<const uint8_t*>(a.bias);
    p.layout = a.grouped_layout;
    p.m = a.m; p.n = a.n; p.k = a.k; p.num_groups = a.num_groups;
    p.lda = lda_b; p.ldb = ldb_b; p.ldd = a.ldd;
    p.bsa = a.batch_stride_a * esz_a; p.bsb = a.batch_stride_b * esz_b; p.bsd = a.batch_stride_d;
    p.sfa_ld = a.sfa_ld; p.sfb_ld = a.sfb_ld; p.sfa_bs = a.sfa_batch_stride; p.sfb_bs = a.sfb_batch_stride;
    const int out_esz = a.d_dtype == DG_DTYPE_F32 ? 4 : a.d_dtype == DG_DTYPE_FP8_E4M3 ? 1 : 2;
    p.gemm_type = a.gemm_type; p.out_esize = out_esz; p.accumulate = a.accumulate != 0;
    p.has_bias = a.bias != nullptr; p.alignment = a.alignment > 0 ? a.alignment : 256;
    p.alpha = a.alpha;
    p.sfd = reinterpret_cast<uint8_t*>(a.sfd);
    p.sfd_ld = a.sfd_ld;
    p.vec_store = (a.ldd % 4 == 0) && ((reinterpret_cast<uintptr_t>(a.d) % (4 * out_esz)) == 0) &&
                  (a.gemm_type != kBatched && a.gemm_type != kMasked ? true : (a.batch_stride_d % 4 == 0));
    p.num_m_blocks = ceil_div(a.m, cfg.bm);
    // anchored tiles (M-grouped psum, BM > 256): a tile row per BM rows plus one per group bounds
    // the tile count; the kernel maps tiles group by group and the spare workgroups exit
    p.anchored = (a.gemm_type == kMGroupedPsum || a.gemm_type == kMGroupedIdx) && tile_anchored(cfg.bm);
    if (p.anchored) p.num_m_blocks += a.gemm_type == kMGroupedIdx ? ceil_div(a.m, p.alignment) : a.num_groups;
    p.num_n_blocks = ceil_div(a.n, cfg.bn);
    p.kbytes_a = (int)kbytes_a; p.kbytes_b = (int)kbytes_b;
    static const int group_m_env = std::getenv("DG_GROUP_M") ? std::atoi(std::getenv("DG_GROUP_M")) : 0;   // tuning
    p.group_m = group_m_env > 0 ? group_m_env : 4;
    const int groups = (a.gemm_type == kBatched || a.gemm_type == kMasked || a.gemm_type == kKGrouped) ? a.num_groups : 1;
    int64_t tiles = plan.skinny_rows ? rows_tiles(a, cfg) : (int64_t)p.num_m_blocks * p.num_n_blocks * groups;
    if (tiles <= 0) return DG_OK;
    // split-K grids are padded to whole groups of 8 tiles (one per XCD); persistent grids hold
    // one workgroup per CU (set_num_sms caps them)
    // (MN-major skinny launches: padded to whole blocks of 8 x the strips that share a 128-byte line of B)
    const int64_t tiles_pad = skinny_mn ? align_up64(tiles, 8 * (a.kind == kBF16 ? 2 : 4)) : tiles;
    int64_t grid = persistent ? std::min<int64_t>(tiles, (int64_t)cus * cfg.occ)
                       : plan.split > 1 ? align_up64(tiles_pad, 8) * plan.split : tiles_pad;
    // Anchored M-grouped tiles under a CU cap: one workgroup per allowed CU walks the layout's real
    // tiles (gemm_walk_kernel).  Uncapped, the upper-bound grid is faster: the dispatcher hands each
    // CU that frees the next real tile and the spare workgroups exit after one scan, where a fixed
    // round-robin walk loses that balance (G=32 routed, alignment 128, cold us: N=4096 K=7168 366
    // vs 346, N=7168 K=2048 217 vs 199; m_indices 407 vs 391, 249 vs 229).  DG_ANCHORED_WALK=1 forces
    // the walk (tuning).
    static const char* walk_env = std::getenv("DG_ANCHORED_WALK");
    const bool walk = p.anchored && !jit && plan.split == 1 &&
                      (cus_capped(cus) || (walk_env != nullptr && walk_env[0] == '1')) &&
                      lookup_walk(a.kind, cfg.bm, cfg.bn, epi_kind) != nullptr;
    if (walk) {
        fn = lookup_walk(a.kind, cfg.bm, cfg.bn, epi_kind);
        grid = std::min<int64_t>(tiles, cus);
    }
    p.a_span = a_span; p.b_span = b_span; p.sfa_span = sfa_span; p.sfb_span = sfb_span;
    if (grid > 0x7fffffffLL) return dg_set_error("dg_gemm: too many tiles");
    p.split_k = plan.split;
    p.split_stages = plan.split_stages;
    p.num_tiles = (int)tiles;
    if (plan.split > 1) {
        // DG_SPLIT_SPREAD=1 (test knob): the splits of a tile run on different XCDs
        const char* spread = std::getenv("DG_SPLIT_SPREAD");
        p.split_spread = spread != nullptr && spread[0] == '1';
        p.counters = reinterpret_cast<int*>(workspace);
        p.ws = reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(workspace) + kCounterBytes);
        p.split_reduce = plan.split_reduce;
    }
    KernelFn reduce_fn = nullptr;
    if (p.split_reduce) {
        reduce_fn = lookup_split_reduce(cfg.bm / 32, cfg.bn / 32, epi_kind);
        if (reduce_fn == nullptr) {
            dg_set_error("dg_gemm: no compiled split-K reduction kernel for this plan");
            return DG_ENOKERNEL;
        }
    }
    int threads = skinny ? plan.skinny_nw * 64 : tile_threads(cfg.bm, cfg.bn);
    unsigned lds_bytes = 0;
    if (gemv_mr > 0) {
        // workgroups of 8 waves / ks rows of B, dealt over the XCDs in contiguous runs
        fn = lookup_gemv(gemv_mr, epi_kind, gemv_waves);
        const int groups_g = a.gemm_type == kBatched ? a.num_groups : 1;
        p.split_k = 1;
        p.split_stages = gemv_ks;
        p.num_n_blocks = ceil_div(a.n, 8 * gemv_waves / gemv_ks);
        const int64_t wgs = (int64_t)p.num_n_blocks * groups_g;
        if (wgs > 0x7ffffff0LL) return dg_set_error("dg_gemm: too many tiles");
        p.num_tiles = (int)wgs;
        tiles = wgs;
        grid = align_up64(wgs, 8);
        threads = gemv_waves * 64;
        lds_bytes = (unsigned)gemv_lds(gemv_mr, a.k, gemv_ks);
    }
    // Under a CU cap (set_num_sms below the device's CUs) at most `cus` workgroups run at a time:
    // one per allowed CU (the reference launches num_cores blocks, csrc/jit_kernels/heuristics.hpp:98).
    // The persistent kernel walks its tiles with that many; the other kernels get the plan's
    // workgroups in stream-ordered launches of at most `cus` each (KParams::vbase; rounded down to
    // whole groups of 8, one per XCD, so the XCD-aware workgroup orders keep their placement), which
    // leaves the kernels' code as it is for uncapped launches.
    p.vgrid = (int)grid;
    p.vbase = 0;
    int64_t launched = grid;
    if (cus_capped(cus) && !persistent && !walk) launched = std::min<int64_t>(grid, cus >= 8 ? cus / 8 * 8 : cus);
    if (info != nullptr) {
        info->plan_workgroups = grid;
        info->block_m = gemv_mr > 0 ? gemv_mr : cfg.bm;
        info->block_n = gemv_mr > 0 ? 8 * gemv_waves / gemv_ks : cfg.bn;
        info->grid = launched;
        info->threads = threads;
        info->tiles = tiles;
        info->split_k = gemv_mr > 0 ? 1 : plan.split;
        info->persistent = persistent || walk ? 1 : 0;
        info->skinny = gemv_mr > 0 ? 3 : skinny ? (plan.skinny_rows ? 2 : 1) : 0;
        info->split_reduce = p.split_reduce;
        return DG_OK;
    }
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    if (a.gemm_type == kMGroupedIdx && !compile_only) {
        // m_indices layout check: a device kernel that sets the sticky DG_ERR_M_INDICES word
        // (no host synchronisation; without the words -- a call that may not allocate, before
        // any other call allocated them -- it checks nothing); for anchored plans the same kernel
        // records each block's valid end for the run table
        int rc = DG_OK;
        if (!p.anchored) {
            rc = check_m_indices(a.grouped_layout, a.m, a.alignment, a.num_groups, st, !noalloc);
            if (rc != DG_OK) return rc;
        } else {
            // the layout's run table, then the per-block valid ends: for dg_gemm_noalloc in its scratch
            // past the split-K tile counters (those must stay zero for the next split-K call; an
            // anchored plan splits no K, so the partial-tile area is free), else in the library's
            // per-stream buffer
            const int64_t nblk = ceil_div(a.m, p.alignment);
            const int64_t need = (1 + 4 * nblk) * 4;
            void* runs = nullptr;
            if (noalloc) {
                if (kCounterBytes + need > a.workspace_bytes)
                    return dg_set_error("dg_gemm_noalloc: m_indices run table exceeds the scratch");
                runs = reinterpret_cast<uint8_t*>(a.workspace) + kCounterBytes;
            } else {
                rc = stream_workspace(st, need, &runs, 1);
                if (rc != DG_OK) return rc;
            }
            int32_t* const table = reinterpret_cast<int32_t*>(runs);
            int32_t* const blk_end = table + 1 + 3 * nblk;
            p.runs = table;
            rc = check_m_indices(a.grouped_layout, a.m, p.alignment, a.num_groups, st, !noalloc, blk_end);
            if (rc != DG_OK) return rc;
            rc = m_indices_runs(a.grouped_layout, a.m, p.alignment, table, blk_end, st);
            if (rc != DG_OK) return rc;
        }
    }
    if (jit) return jit_run(a, cfg, epi_kind, plan.split, p, launched, st, compile_only);
    for (int64_t base = 0; base < grid; base += launched) {
        p.vbase = (int)base;
        const unsigned n = (unsigned)std::min<int64_t>(launched, grid - base);
        const hipError_t e = launch_module_kernel(reinterpret_cast<const void*>(fn), n, (unsigned)threads, p, st, lds_bytes);
        if (e != hipSuccess) {
            dg_set_error(hipGetErrorString(e));
            return DG_ELAUNCH;
        }
        if (persistent || walk) break;   // (one launch walks every tile)
    }
    if (reduce_fn != nullptr) {
        // second launch: one wave per 32x32 block of the tiles, DG_REDUCE_WAVES (tuning, default 1) per workgroup
        static const int rw_env = std::getenv("DG_REDUCE_WAVES") ? std::atoi(std::getenv("DG_REDUCE_WAVES")) : 1;
        const int rw = rw_env == 2 || rw_env == 4 ? rw_env : 1;
        const int64_t rgrid = ceil_div(tiles * (cfg.bm / 32) * (cfg.bn / 32), rw);
        const int64_t rlaunched = cus_capped(cus) ? std::min<int64_t>(rgrid, cus >= 8 ? cus / 8 * 8 : cus) : rgrid;
        p.vgrid = (int)rgrid;
        for (int64_t base = 0; base < rgrid; base += rlaunched) {
            p.vbase = (int)base;
            const unsigned n = (unsigned)std::min<int64_t>(rlaunched, rgrid - base);
            const hipError_t e = launch_module_kernel(reinterpret_cast<const void*>(reduce_fn), n, 64u * rw, p, st, 0);
            if (e != hipSuccess) {
                dg_set_error(hipGetErrorString(e));
                return DG_ELAUNCH;
            }
        }
    }
    return DG_OK;
}

}  // namespace

extern "C" int dg_gemm(const dg_gemm_args* args, void* stream) { return gemm_impl(args, stream, false); }

extern "C" int dg_stream_workspace(void* stream, void** ptr, int64_t* bytes) {
    if (ptr == nullptr || bytes == nullptr) return dg_set_error("dg_stream_workspace: null argument");
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return dg_set_error("dg_stream_workspace: no current HIP device");
    std::lock_guard<std::mutex> lk(g_stream_ws_mu);
    auto it = g_stream_ws.find({dev, reinterpret_cast<hipStream_t>(stream), 0});
    *ptr = it == g_stream_ws.end() ? nullptr : it->second.ptr;
    *bytes = it == g_stream_ws.end() ? 0 : it->second.bytes;
    return DG_OK;
}

// ---------------------------------------------------------------------------------------------
// dg_gemm_noalloc: dg_gemm with the split-K workspace taken from a fixed device array instead of
// the caller's (for callers that cannot allocate: graph capture, serving loops).
namespace {

// Scratch of dg_gemm_noalloc: the workspace layout of dg_gemm (64 KiB of tile counters, then the
// fp32 partial tiles).  Zero at load; every launch leaves the counters zero again.  Each device
// holds its own copy until the process ends.
constexpr int64_t kNoAllocScratchBytes = (16 << 20) + dg::kCounterBytes;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

std::mutex g_scratch_mu;
void* g_scratch_ptr[64] = {nullptr};

// Device address of `scratch` on the current device (host code never passes the array's name:
// that is a host-side stand-in, not a device address).
int scratch_address(void** out) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64)
        return dg_set_error("dg_gemm_noalloc: no current HIP device");
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (g_scratch_ptr[dev] == nullptr) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || p == nullptr) {
            std::string msg = std::string("dg_gemm_noalloc: hipGetSymbolAddress(scratch) failed: ") + hipGetErrorString(e);
            dg_set_error(msg.c_str());
            return DG_ELAUNCH;
        }
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return DG_OK;
}

}  // namespace

extern "C" int dg_gemm_noalloc(const dg_gemm_args* args, void* stream) {
    if (args == nullptr) return dg_set_error("dg_gemm_noalloc: null args");
    dg_gemm_args a = *args;
    if (a.workspace != nullptr || a.workspace_bytes != 0 || a.library_workspace != 0)
        return dg_set_error("dg_gemm_noalloc: the library provides the workspace (pass workspace = NULL, 0 bytes, "
                            "library_workspace = 0)");
    int64_t need = 0;
    a.workspace = reinterpret_cast<void*>(1);   // (any non-null value: the plan may then split K)
    int rc = dg_gemm_workspace_size(&a, &need);
    if (rc != DG_OK) return rc;
    if (need > kNoAllocScratchBytes) {
        char buf[200];
        snprintf(buf, sizeof(buf), "dg_gemm_noalloc: this problem's split-K plan needs %lld bytes of scratch, more than "
                 "the %lld-byte maximum (call dg_gemm with a workspace, or split_k = 1)", (long long)need,
                 (long long)kNoAllocScratchBytes);
        return dg_set_error(buf);
    }
    // (the scratch stands in for a workspace whether or not this plan splits K, so the plan is
    // always the one dg_gemm makes when given a workspace)
    void* ptr = nullptr;
    rc = scratch_address(&ptr);
    if (rc != DG_OK) return rc;
    a.workspace = ptr;
    a.workspace_bytes = kNoAllocScratchBytes;
    return gemm_impl(&a, stream, false, nullptr, true);
}

extern "C" int dg_launch_plan(const dg_gemm_args* args, dg_launch_info* info) {
    if (args == nullptr || info == nullptr) return dg_set_error("dg_launch_plan: null argument");
    return gemm_impl(args, nullptr, true, info);
}

extern "C" int dg_jit_compile(const dg_gemm_args* args) {
    if (args == nullptr) return dg_set_error("dg_jit_compile: null args");
    dg_gemm_args a = *args;
    a.jit = 1;
    return gemm_impl(&a, nullptr, true);
}
