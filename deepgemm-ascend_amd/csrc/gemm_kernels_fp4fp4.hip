// Instantiates the GEMM kernel for every tile shape of the menu (kFP4FP4 operands).
#include "gemm_tiles.hpp"

namespace dg {
KernelFn lookup_kernel_fp4fp4(int bm, int bn, int epi, bool persistent) { return lookup_tile<kFP4FP4>(bm, bn, epi, persistent); }
}  // namespace dg
