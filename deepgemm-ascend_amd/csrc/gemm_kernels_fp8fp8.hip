// Instantiates the GEMM kernel for every tile shape of the menu (kFP8FP8 operands).
#include "gemm_tiles.hpp"

namespace dg {
KernelFn lookup_kernel_fp8fp8(int bm, int bn, int epi, bool persistent) { return lookup_tile<kFP8FP8>(bm, bn, epi, persistent); }
KernelFn lookup_walk_fp8fp8(int bm, int bn, int epi) { return lookup_walk<kFP8FP8>(bm, bn, epi); }
}  // namespace dg
