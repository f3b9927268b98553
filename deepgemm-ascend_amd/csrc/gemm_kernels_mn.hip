// Instantiates the tile kernel with MN-major operands (e4m3 x e4m3 and bf16 x bf16, the 128-byte-stage
// tiles of at most 256 x 256): A, B or both read in place from [K][MN] storage (csrc/gemm_kernel.hpp,
// AMN / BMN).
#include "gemm_tiles.hpp"

namespace dg {
namespace {

template <int I, int KIND, bool AMN, bool BMN>
KernelFn mn_epi(int epi) {
    constexpr TileCfg t = kTiles[I];
    // (the anchored 384-row tiles leave no LDS for a 256-element MN-major B row)
    if constexpr (t.km != 2 || t.stages != 2 || t.bm > 256 || t.bn > 256) {
        return nullptr;
    } else {
        switch (epi) {
            case kEpiF32: return &gemm_kernel<t.bm, t.bn, t.wgm, t.nw, t.lw, t.stages, t.km, t.occ, KIND, kEpiF32, AMN, BMN>;
            case kEpiBf16: return &gemm_kernel<t.bm, t.bn, t.wgm, t.nw, t.lw, t.stages, t.km, t.occ, KIND, kEpiBf16, AMN, BMN>;
            case kEpiBf16SR: return &gemm_kernel<t.bm, t.bn, t.wgm, t.nw, t.lw, t.stages, t.km, t.occ, KIND, kEpiBf16SR, AMN, BMN>;
            case kEpiFp8:
                if constexpr (KIND == kFP8FP8) return &gemm_kernel<t.bm, t.bn, t.wgm, t.nw, t.lw, t.stages, t.km, t.occ, KIND, kEpiFp8, AMN, BMN>;
                else return nullptr;
            default: return nullptr;
        }
    }
}

template <int KIND, int I = 0>
KernelFn mn_find(int bm, int bn, int epi, bool amn, bool bmn) {
    if constexpr (I == kNumTiles) {
        return nullptr;
    } else {
        if (bm == kTiles[I].bm && bn == kTiles[I].bn) {
            if (amn && bmn) return mn_epi<I, KIND, true, true>(epi);
            if (amn) return mn_epi<I, KIND, true, false>(epi);
            if (bmn) return mn_epi<I, KIND, false, true>(epi);
            return nullptr;
        }
        return mn_find<KIND, I + 1>(bm, bn, epi, amn, bmn);
    }
}

}  // namespace

KernelFn lookup_kernel_mn(int kind, int bm, int bn, int epi, bool a_mn, bool b_mn) {
    switch (kind) {
        case kFP8FP8: return mn_find<kFP8FP8>(bm, bn, epi, a_mn, b_mn);
        case kBF16: return mn_find<kBF16>(bm, bn, epi, a_mn, b_mn);
        default: return nullptr;
    }
}

}  // namespace dg
