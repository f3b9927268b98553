// Instantiates the skinny-M kernel (csrc/skinny_kernel.hpp) for every configuration of the
// kSkinny menu, operand kind and epilogue.
#include "gemm_tiles.hpp"
#include "skinny_kernel.hpp"

namespace dg {
namespace {

template <int I, int KIND>
KernelFn skinny_epi(int epi) {
    constexpr SkinnyCfg c = kSkinny[I];
    switch (epi) {
        case kEpiF32: return &skinny_kernel<KIND, c.mt, c.nb, c.nw, c.d, c.ar, kEpiF32>;
        case kEpiBf16: return &skinny_kernel<KIND, c.mt, c.nb, c.nw, c.d, c.ar, kEpiBf16>;
        case kEpiBf16SR: return &skinny_kernel<KIND, c.mt, c.nb, c.nw, c.d, c.ar, kEpiBf16SR>;
        case kEpiFp8:
            if constexpr (KIND == kFP8FP8) return &skinny_kernel<KIND, c.mt, c.nb, c.nw, c.d, c.ar, kEpiFp8>;
            else return nullptr;
        default: return nullptr;
    }
}

template <int KIND, int I = 0>
KernelFn skinny_find(int mt, int nb, int nw, int d, int ar, int epi) {
    if constexpr (I == kNumSkinny) {
        return nullptr;
    } else {
        if (mt == kSkinny[I].mt && nb == kSkinny[I].nb && nw == kSkinny[I].nw && d == kSkinny[I].d && ar == kSkinny[I].ar)
            return skinny_epi<I, KIND>(epi);
        return skinny_find<KIND, I + 1>(mt, nb, nw, d, ar, epi);
    }
}

template <int I, int KIND>
KernelFn rows_epi(int epi) {
    constexpr SkinnyRowsCfg c = kSkinnyRows[I];
    switch (epi) {
        case kEpiF32: return &skinny_rows_kernel<KIND, c.mt, c.nb, c.d, kEpiF32>;
        case kEpiBf16: return &skinny_rows_kernel<KIND, c.mt, c.nb, c.d, kEpiBf16>;
        case kEpiBf16SR: return &skinny_rows_kernel<KIND, c.mt, c.nb, c.d, kEpiBf16SR>;
        case kEpiFp8:
            if constexpr (KIND == kFP8FP8) return &skinny_rows_kernel<KIND, c.mt, c.nb, c.d, kEpiFp8>;
            else return nullptr;
        default: return nullptr;
    }
}

template <int KIND, int I = 0>
KernelFn rows_find(int mt, int nb, int d, int epi) {
    if constexpr (I == kNumSkinnyRows) {
        return nullptr;
    } else {
        if (mt == kSkinnyRows[I].mt && nb == kSkinnyRows[I].nb && d == kSkinnyRows[I].d) return rows_epi<I, KIND>(epi);
        return rows_find<KIND, I + 1>(mt, nb, d, epi);
    }
}

template <int I>
KernelFn reduce_epi(int epi) {
    constexpr SkinnyRowsCfg c = kSkinnyRows[I];
    switch (epi) {
        case kEpiF32: return &split_reduce_kernel<c.mt, c.nb, kEpiF32>;
        case kEpiBf16: return &split_reduce_kernel<c.mt, c.nb, kEpiBf16>;
        case kEpiBf16SR: return &split_reduce_kernel<c.mt, c.nb, kEpiBf16SR>;
        case kEpiFp8: return &split_reduce_kernel<c.mt, c.nb, kEpiFp8>;
        default: return nullptr;
    }
}

template <int I = 0>
KernelFn reduce_find(int mt, int nb, int epi) {
    if constexpr (I == kNumSkinnyRows) {
        return nullptr;
    } else {
        if (mt == kSkinnyRows[I].mt && nb == kSkinnyRows[I].nb) return reduce_epi<I>(epi);
        return reduce_find<I + 1>(mt, nb, epi);
    }
}

}  // namespace

KernelFn lookup_split_reduce(int mt, int nb, int epi) { return reduce_find(mt, nb, epi); }

KernelFn lookup_skinny_rows(int kind, int mt, int nb, int d, int epi) {
    switch (kind) {
        case kFP8FP8: return rows_find<kFP8FP8>(mt, nb, d, epi);
        case kFP8FP4: return rows_find<kFP8FP4>(mt, nb, d, epi);
        case kFP4FP4: return rows_find<kFP4FP4>(mt, nb, d, epi);
        case kBF16: return rows_find<kBF16>(mt, nb, d, epi);
        default: return nullptr;
    }
}

KernelFn lookup_skinny(int kind, int mt, int nb, int nw, int d, int ar, int epi) {
    switch (kind) {
        case kFP8FP8: return skinny_find<kFP8FP8>(mt, nb, nw, d, ar, epi);
        case kFP8FP4: return skinny_find<kFP8FP4>(mt, nb, nw, d, ar, epi);
        case kFP4FP4: return skinny_find<kFP4FP4>(mt, nb, nw, d, ar, epi);
        case kBF16: return skinny_find<kBF16>(mt, nb, nw, d, ar, epi);
        default: return nullptr;
    }
}

}  // namespace dg
