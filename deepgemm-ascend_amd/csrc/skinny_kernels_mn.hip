// Instantiates the skinny-M kernel (csrc/skinny_kernel.hpp) with MN-major B (stored [K][N], read in
// place) for the 32-column configurations of the kSkinny menu, e4m3 x e4m3 and bf16 x bf16.
#include "gemm_tiles.hpp"
#include "skinny_kernel.hpp"

namespace dg {
namespace {

template <int I, int KIND>
KernelFn skinny_mn_epi(int epi) {
    constexpr SkinnyCfg c = kSkinny[I];
    if constexpr (c.nb != 1) {
        return nullptr;
    } else {
        switch (epi) {
            case kEpiF32: return &skinny_kernel<KIND, c.mt, c.nb, c.nw, c.d, c.ar, kEpiF32, true>;
            case kEpiBf16: return &skinny_kernel<KIND, c.mt, c.nb, c.nw, c.d, c.ar, kEpiBf16, true>;
            case kEpiBf16SR: return &skinny_kernel<KIND, c.mt, c.nb, c.nw, c.d, c.ar, kEpiBf16SR, true>;
            case kEpiFp8:
                if constexpr (KIND == kFP8FP8) return &skinny_kernel<KIND, c.mt, c.nb, c.nw, c.d, c.ar, kEpiFp8, true>;
                else return nullptr;
            default: return nullptr;
        }
    }
}

template <int KIND, int I = 0>
KernelFn skinny_mn_find(int mt, int nb, int nw, int d, int ar, int epi) {
    if constexpr (I == kNumSkinny) {
        return nullptr;
    } else {
        if (mt == kSkinny[I].mt && nb == kSkinny[I].nb && nw == kSkinny[I].nw && d == kSkinny[I].d && ar == kSkinny[I].ar)
            return skinny_mn_epi<I, KIND>(epi);
        return skinny_mn_find<KIND, I + 1>(mt, nb, nw, d, ar, epi);
    }
}

}  // namespace

KernelFn lookup_skinny_mn(int kind, int mt, int nb, int nw, int d, int ar, int epi) {
    switch (kind) {
        case kFP8FP8: return skinny_mn_find<kFP8FP8>(mt, nb, nw, d, ar, epi);
        case kBF16: return skinny_mn_find<kBF16>(mt, nb, nw, d, ar, epi);
        default: return nullptr;
    }
}

}  // namespace dg
