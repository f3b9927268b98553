// Menu of compiled tile shapes and the per-kind kernel lookup tables.
#pragma once

#include "gemm_kernel.hpp"
#include "gemm_persistent.hpp"
#include "../../include/deep_gemm_amd.h"

namespace dg {

using KernelFn = void (*)(const KParams);

// epi: kEpiF32, kEpiBf16, kEpiBf16SR or kEpiFp8 (see gemm_kernel.hpp)

struct TileCfg {
    int bm, bn;
    int wgm;      // waves along M (nw / wgm along N)
    int nw;       // waves per workgroup: 8 = two per SIMD, so one wave's MFMAs issue while the
                  // other waits on loads; 4 where a 4-wave tile needs more than 256 registers
    int lw;       // waves that issue the global->LDS loads (nw, or 4 of 8)
    int stages;   // depth of the LDS ring (deeper for small tiles to keep more bytes in flight
                  // per CU)
    int km;       // MFMA K-steps per stage: 2 = 128-byte fp8 rows (whole-line loads), 1 = 64
    int occ;      // workgroups per CU (2: LDS ring and registers sized for two co-resident
                  // workgroups, whose prologues and epilogues then overlap each other's main loops)
    int stage_cycles;   // measured cycles per 64 K with every CU busy (fp8, MI355X)
    int nsb = 0;        // 3: B rows get a ring of three slots beside the two of A + SF, where that fits
                        // the LDS for the kind (0: one shared ring)
};

// Measured on MI355X (fp8, cold L2): 4096x7168x2048 256x224 70 us, 256x256 72 us; 4096x2112x7168 256x160
// (224 tiles, one round at 88% of the CUs) 84.8 us, 256x224 (160 tiles) 91.9 us; M-grouped contiguous (32
// experts, ~257 rows each, alignment 128) N=4096 K=7168: 128x256 as 8 waves / one workgroup per CU 572 us, as
// 4 waves / two workgroups per CU 509 us; skinny M=128, N=7168, K=16384: 128x128 split 4 57 us.
constexpr TileCfg kTiles[] = {
    {256, 256, 4, 8, 4, 2, 2, 1, 1380, 3}, {256, 224, 4, 8, 4, 2, 2, 1, 1250, 3}, {256, 128, 4, 8, 8, 4, 1, 1, 937},
    {128, 256, 2, 4, 4, 3, 1, 2, 985},  {128, 128, 2, 4, 4, 4, 1, 1, 1056}, {64, 128, 2, 4, 4, 6, 1, 2, 588},
    {32, 128, 1, 4, 4, 6, 1, 2, 643},  {256, 160, 4, 8, 4, 2, 2, 1, 950, 3},
    // tiles anchored at each group's first row (M-grouped psum layouts only)
    {384, 192, 4, 8, 8, 2, 2, 1, 1250}, {384, 128, 4, 8, 4, 2, 2, 1, 1000},
};
constexpr int kNumTiles = sizeof(kTiles) / sizeof(kTiles[0]);

// Split-K runs on tiles whose waves split N into equal 32-column multiples (a ragged tile --
// 256x224 over two wave columns: 128 + 96 -- keeps no split-K partial layout).
constexpr bool tile_splittable(const TileCfg& t) { return t.nw == 0 || (t.bn / (t.nw / t.wgm)) % 32 == 0; }

template <int I, int KIND>
KernelFn pick_epi(int epi) {
    constexpr TileCfg t = kTiles[I];
    switch (epi) {
        case kEpiF32: return &gemm_kernel<t.bm, t.bn, t.wgm, t.nw, t.lw, t.stages, t.km, t.occ, KIND, kEpiF32, false, false, t.nsb>;
        case kEpiBf16: return &gemm_kernel<t.bm, t.bn, t.wgm, t.nw, t.lw, t.stages, t.km, t.occ, KIND, kEpiBf16, false, false, t.nsb>;
        case kEpiBf16SR: return &gemm_kernel<t.bm, t.bn, t.wgm, t.nw, t.lw, t.stages, t.km, t.occ, KIND, kEpiBf16SR, false, false, t.nsb>;
        case kEpiFp8:
            // FP8 output exists for e4m3 x e4m3 batched / dense GEMMs only (fp8_bmm)
            if constexpr (KIND == kFP8FP8) return &gemm_kernel<t.bm, t.bn, t.wgm, t.nw, t.lw, t.stages, t.km, t.occ, KIND, kEpiFp8, false, false, t.nsb>;
            else return nullptr;
        default: return nullptr;
    }
}

// Persistent kernels exist for the 128-K-stage (km = 2, two-slot ring) tiles of up to 256 rows, except
// 256x256, whose persistent body does not fit the register file (the planner never takes it).
template <int I, int KIND>
KernelFn pick_persistent_epi(int epi) {
    constexpr TileCfg t = kTiles[I];
    if constexpr (t.km != 2 || t.stages != 2 || t.bm > 256 || (t.bm == 256 && t.bn == 256)) {
        return nullptr;
    } else {
        switch (epi) {
            case kEpiF32: return &gemm_persistent_kernel<t.bm, t.bn, t.wgm, t.nw, t.lw, t.occ, KIND, kEpiF32>;
            case kEpiBf16: return &gemm_persistent_kernel<t.bm, t.bn, t.wgm, t.nw, t.lw, t.occ, KIND, kEpiBf16>;
            case kEpiBf16SR: return &gemm_persistent_kernel<t.bm, t.bn, t.wgm, t.nw, t.lw, t.occ, KIND, kEpiBf16SR>;
            case kEpiFp8:
                if constexpr (KIND == kFP8FP8) return &gemm_persistent_kernel<t.bm, t.bn, t.wgm, t.nw, t.lw, t.occ, KIND, kEpiFp8>;
                else return nullptr;
            default: return nullptr;
        }
    }
}

// Persistent walk kernels exist for the anchored (M-grouped, more than 256 rows) tiles.
template <int I, int KIND>
KernelFn pick_walk_epi(int epi) {
    constexpr TileCfg t = kTiles[I];
    if constexpr (t.bm <= 256) {
        return nullptr;
    } else {
        switch (epi) {
            case kEpiF32: return &gemm_walk_kernel<t.bm, t.bn, t.wgm, t.nw, t.lw, t.stages, t.km, t.occ, KIND, kEpiF32, t.nsb>;
            case kEpiBf16: return &gemm_walk_kernel<t.bm, t.bn, t.wgm, t.nw, t.lw, t.stages, t.km, t.occ, KIND, kEpiBf16, t.nsb>;
            default: return nullptr;
        }
    }
}

template <int KIND, int I = 0>
KernelFn lookup_walk(int bm, int bn, int epi) {
    if constexpr (I == kNumTiles) {
        return nullptr;
    } else {
        if (bm == kTiles[I].bm && bn == kTiles[I].bn) return pick_walk_epi<I, KIND>(epi);
        return lookup_walk<KIND, I + 1>(bm, bn, epi);
    }
}

template <int KIND, int I = 0>
KernelFn lookup_tile(int bm, int bn, int epi, bool persistent) {
    if constexpr (I == kNumTiles) {
        return nullptr;
    } else {
        if (bm == kTiles[I].bm && bn == kTiles[I].bn)
            return persistent ? pick_persistent_epi<I, KIND>(epi) : pick_epi<I, KIND>(epi);
        return lookup_tile<KIND, I + 1>(bm, bn, epi, persistent);
    }
}

// Threads per workgroup of the (bm, bn) kernel (0 if not in the menu).
inline int tile_threads(int bm, int bn) {
    for (const TileCfg& t : kTiles)
        if (t.bm == bm && t.bn == bn) return t.nw * 64;
    return 0;
}

// Run-time compiled kernel of one launch plan (csrc/jit.hip): compile or fetch it and, unless
// compile_only, launch it on `st`.
int jit_run(const dg_gemm_args& a, const TileCfg& cfg, int epi, int split, const KParams& p, int64_t grid,
            hipStream_t st, bool compile_only);

// Skinny-M kernels (csrc/skinny_kernel.hpp): strips of 32 nb columns, M <= ar (<= 32 mt) rows of
// A, nw waves splitting K, each with a ring of d group slots.
struct SkinnyCfg {
    int mt, nb, nw, d, ar;
};
constexpr SkinnyCfg kSkinny[] = {{1, 1, 4, 2, 16}, {1, 1, 4, 3, 16}, {1, 1, 4, 2, 32}, {1, 1, 4, 3, 32},
                                 {1, 1, 8, 2, 16}, {1, 2, 4, 2, 16}, {2, 1, 4, 2, 64},
                                 {4, 1, 4, 2, 128}};
constexpr int kNumSkinny = sizeof(kSkinny) / sizeof(kSkinny[0]);
KernelFn lookup_skinny(int kind, int mt, int nb, int nw, int d, int ar, int epi);
// the same with MN-major B (stored [K][N], read in place): e4m3 / bf16, 32-column strips (nb = 1)
KernelFn lookup_skinny_mn(int kind, int mt, int nb, int nw, int d, int ar, int epi);

// Shared-ring decode kernels (skinny_rows_kernel): MT x NB waves, one 32x32 block each, a ring
// of d group slots shared by the workgroup.
struct SkinnyRowsCfg {
    int mt, nb, d;
};
constexpr SkinnyRowsCfg kSkinnyRows[] = {{4, 1, 3}, {4, 1, 4}, {4, 1, 5}, {4, 2, 4}, {4, 4, 4}, {2, 1, 4}, {2, 2, 4}, {2, 4, 4}};
constexpr int kNumSkinnyRows = sizeof(kSkinnyRows) / sizeof(kSkinnyRows[0]);
KernelFn lookup_skinny_rows(int kind, int mt, int nb, int d, int epi);
// second launch of a split-K shared-ring plan: sums the partials of each 32x32 block, then its epilogue
KernelFn lookup_split_reduce(int mt, int nb, int epi);

// Decode GEMV kernels (csrc/gemv_kernel.hip): e4m3 x e4m3, M <= mr (1, 2, 4), fp32 / bf16 D;
// whole rows of B per wave, A staged in LDS as f16 (gemv_lds(mr, k, rows per wave) bytes).
KernelFn lookup_gemv(int mr, int epi, int waves);   // waves per workgroup: 4 or 8
int gemv_lds(int mr, int k, int rpw);

KernelFn lookup_kernel_fp8fp8(int bm, int bn, int epi, bool persistent);
// anchored M-grouped tiles walked persistently (gemm_walk_kernel), e4m3 x e4m3 / bf16
KernelFn lookup_walk_fp8fp8(int bm, int bn, int epi);
KernelFn lookup_walk_bf16(int bm, int bn, int epi);
KernelFn lookup_kernel_fp8fp4(int bm, int bn, int epi, bool persistent);
KernelFn lookup_kernel_fp4fp4(int bm, int bn, int epi, bool persistent);
KernelFn lookup_kernel_bf16(int bm, int bn, int epi, bool persistent);
// e4m3 x e4m3 and bf16 x bf16 tile kernels reading MN-major A and / or B in place (the 128-byte-stage
// tiles of at most 256 x 256; nullptr otherwise)
KernelFn lookup_kernel_mn(int kind, int bm, int bn, int epi, bool a_mn, bool b_mn);

}  // namespace dg
