// Menu of compiled tile shapes and the per-kind kernel lookup tables.
#pragma once

#include "gemm_kernel.hpp"

namespace dg {

using KernelFn = void (*)(const KParams);

// epi: kEpiF32 or kEpiBf16 (see gemm_kernel.hpp)

struct TileCfg {
    int bm, bn;
};

// Tile shapes compiled for every operand kind (BM x BN, 4 waves in 2 x 2).
constexpr TileCfg kTiles[] = {{256, 256}, {256, 224}, {256, 128}, {128, 256},
                              {128, 128}, {64, 128},  {32, 128}};
constexpr int kNumTiles = sizeof(kTiles) / sizeof(kTiles[0]);

#define DG_TILE_TABLE(KIND_)                                          \
    if (bm == 256 && bn == 256) return epi == kEpiF32 ? &gemm_kernel<256, 256, KIND_, kEpiF32> : &gemm_kernel<256, 256, KIND_, kEpiBf16>; \
    if (bm == 256 && bn == 224) return epi == kEpiF32 ? &gemm_kernel<256, 224, KIND_, kEpiF32> : &gemm_kernel<256, 224, KIND_, kEpiBf16>; \
    if (bm == 256 && bn == 128) return epi == kEpiF32 ? &gemm_kernel<256, 128, KIND_, kEpiF32> : &gemm_kernel<256, 128, KIND_, kEpiBf16>; \
    if (bm == 128 && bn == 256) return epi == kEpiF32 ? &gemm_kernel<128, 256, KIND_, kEpiF32> : &gemm_kernel<128, 256, KIND_, kEpiBf16>; \
    if (bm == 128 && bn == 128) return epi == kEpiF32 ? &gemm_kernel<128, 128, KIND_, kEpiF32> : &gemm_kernel<128, 128, KIND_, kEpiBf16>; \
    if (bm == 64 && bn == 128) return epi == kEpiF32 ? &gemm_kernel<64, 128, KIND_, kEpiF32> : &gemm_kernel<64, 128, KIND_, kEpiBf16>;   \
    if (bm == 32 && bn == 128) return epi == kEpiF32 ? &gemm_kernel<32, 128, KIND_, kEpiF32> : &gemm_kernel<32, 128, KIND_, kEpiBf16>;   \
    return nullptr;

KernelFn lookup_kernel_fp8fp8(int bm, int bn, int epi);
KernelFn lookup_kernel_fp8fp4(int bm, int bn, int epi);
KernelFn lookup_kernel_fp4fp4(int bm, int bn, int epi);
KernelFn lookup_kernel_bf16(int bm, int bn, int epi);

}  // namespace dg
