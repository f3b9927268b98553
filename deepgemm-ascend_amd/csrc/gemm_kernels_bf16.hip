// Instantiates the GEMM kernel for every tile shape of the menu (kBF16 operands).
#include "gemm_tiles.hpp"

namespace dg {
KernelFn lookup_kernel_bf16(int bm, int bn, int epi, bool persistent) { return lookup_tile<kBF16>(bm, bn, epi, persistent); }
KernelFn lookup_walk_bf16(int bm, int bn, int epi) { return lookup_walk<kBF16>(bm, bn, epi); }
}  // namespace dg
