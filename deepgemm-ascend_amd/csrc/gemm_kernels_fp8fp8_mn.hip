// Instantiates the tile kernel with MN-major operands (e4m3 x e4m3, the 128-K-stage tiles of at most
// 256 x 256): A, B or both read in place from [K][MN] storage (csrc/gemm_kernel.hpp, AMN / BMN).
#include "gemm_tiles.hpp"

namespace dg {
namespace {

template <int I, bool AMN, bool BMN>
KernelFn mn_epi(int epi) {
    constexpr TileCfg t = kTiles[I];
    if constexpr (t.km != 2 || t.stages != 2 || t.bm > 256 || t.bn > 256) {
        return nullptr;
    } else {
        switch (epi) {
            case kEpiF32: return &gemm_kernel<t.bm, t.bn, t.wgm, t.nw, t.lw, t.stages, t.km, t.occ, kFP8FP8, kEpiF32, AMN, BMN>;
            case kEpiBf16: return &gemm_kernel<t.bm, t.bn, t.wgm, t.nw, t.lw, t.stages, t.km, t.occ, kFP8FP8, kEpiBf16, AMN, BMN>;
            case kEpiBf16SR: return &gemm_kernel<t.bm, t.bn, t.wgm, t.nw, t.lw, t.stages, t.km, t.occ, kFP8FP8, kEpiBf16SR, AMN, BMN>;
            case kEpiFp8: return &gemm_kernel<t.bm, t.bn, t.wgm, t.nw, t.lw, t.stages, t.km, t.occ, kFP8FP8, kEpiFp8, AMN, BMN>;
            default: return nullptr;
        }
    }
}

template <int I = 0>
KernelFn mn_find(int bm, int bn, int epi, bool amn, bool bmn) {
    if constexpr (I == kNumTiles) {
        return nullptr;
    } else {
        if (bm == kTiles[I].bm && bn == kTiles[I].bn) {
            if (amn && bmn) return mn_epi<I, true, true>(epi);
            if (amn) return mn_epi<I, true, false>(epi);
            if (bmn) return mn_epi<I, false, true>(epi);
            return nullptr;
        }
        return mn_find<I + 1>(bm, bn, epi, amn, bmn);
    }
}

}  // namespace

KernelFn lookup_kernel_fp8fp8_mn(int bm, int bn, int epi, bool a_mn, bool b_mn) { return mn_find(bm, bn, epi, a_mn, b_mn); }

}  // namespace dg
