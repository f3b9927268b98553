// MN-major -> K-major operand copy (HBM-bound byte work).
//
// The GEMM kernels stream K-major operand rows; an operand the caller holds MN-major (the `tn`
// / `nn` / `tt` layouts, the K-grouped wgrad operands [Ktot, M], einsum views whose contraction
// axis is not the innermost) is transposed once on the device.  One workgroup moves a 64 (K) x
// 64 (MN) element tile: coalesced 16-byte global loads along MN into a padded LDS tile, then
// 16-byte global stores along K.  Columns K .. k_padded-1 of the output are written as zeros
// so the result is directly a 16-byte-aligned K-major operand.
#include "dg_common.hpp"
#include "../../include/deep_gemm_amd.h"

namespace dg {

struct TransposeParams {
    const uint8_t* src;
    uint8_t* dst;
    int64_t src_bs, src_ld, dst_bs, dst_ld;   // elements
    int k, mn, k_padded;
};

template <int E>   // element bytes: 1 (e4m3 / int8) or 2 (bf16)
__global__ __launch_bounds__(256) void transpose_to_k_major_kernel(const TransposeParams p) {
    constexpr int T = 64;                 // tile edge in elements
    constexpr int ROWB = T * E;           // bytes of one tile row
    constexpr int PAD = 4;                // LDS row padding (bytes) against bank conflicts
    constexpr int VEC = 16 / E;           // elements per 16-byte access
    constexpr int TPR = T / VEC;          // threads per tile row
    constexpr int RPP = 256 / TPR;        // rows per pass
    __shared__ __align__(16) uint8_t tile[T][ROWB + PAD];

    const int tid = threadIdx.x;
    const int k0 = blockIdx.x * T, mn0 = blockIdx.y * T, b = blockIdx.z;
    const uint8_t* src = p.src + ((int64_t)b * p.src_bs) * E;
    uint8_t* dst = p.dst + ((int64_t)b * p.dst_bs) * E;

    // load: tile row = one K index, 64 MN elements
    const int c = (tid % TPR) * VEC;
    const bool vec_ok = (p.src_ld % VEC) == 0 && (reinterpret_cast<uintptr_t>(src) % 16) == 0;
#pragma unroll
    for (int r0 = 0; r0 < T; r0 += RPP) {
        const int r = r0 + tid / TPR;
        const int k = k0 + r, mn = mn0 + c;
        uint32_t w[4] = {0, 0, 0, 0};
        if (k < p.k) {
            const uint8_t* s = src + ((int64_t)k * p.src_ld + mn) * E;
            if (vec_ok && mn + VEC <= p.mn) {
                const i32x4 v = *reinterpret_cast<const i32x4*>(s);
                w[0] = v[0]; w[1] = v[1]; w[2] = v[2]; w[3] = v[3];
            } else {
                uint8_t* wb = reinterpret_cast<uint8_t*>(w);
                for (int i = 0; i < VEC; ++i)
                    if (mn + i < p.mn)
                        for (int e = 0; e < E; ++e) wb[i * E + e] = s[i * E + e];
            }
        }
        uint32_t* t = reinterpret_cast<uint32_t*>(&tile[r][c * E]);
        t[0] = w[0]; t[1] = w[1]; t[2] = w[2]; t[3] = w[3];
    }
    __syncthreads();

    // store: output row = one MN index, 64 K elements (zeros past K up to k_padded)
#pragma unroll
    for (int r0 = 0; r0 < T; r0 += RPP) {
        const int r = r0 + tid / TPR;          // MN within the tile
        const int mn = mn0 + r, k = k0 + c;    // first K of this thread's 16 bytes
        if (mn >= p.mn || k >= p.k_padded) continue;
        uint32_t w[4];
        uint8_t* wb = reinterpret_cast<uint8_t*>(w);
#pragma unroll
        for (int i = 0; i < VEC; ++i)
#pragma unroll
            for (int e = 0; e < E; ++e) wb[i * E + e] = tile[c + i][r * E + e];
        uint8_t* d = dst + ((int64_t)mn * p.dst_ld + k) * E;
        if (k + VEC <= p.k_padded) {
            *reinterpret_cast<i32x4*>(d) = i32x4{(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
        } else {
            for (int i = 0; i < VEC && k + i < p.k_padded; ++i)
                for (int e = 0; e < E; ++e) d[i * E + e] = wb[i * E + e];
        }
    }
}

}  // namespace dg

extern "C" __attribute__((visibility("hidden"))) int dg_set_error(const char* msg);

extern "C" int dg_transpose_to_k_major(const void* src, int32_t elem_bytes, int32_t batches, int64_t src_batch_stride,
                                       int64_t src_ld, int32_t k, int32_t mn, void* dst, int64_t dst_batch_stride,
                                       int64_t dst_ld, int32_t k_padded, void* stream) {
    using namespace dg;
    if (src == nullptr || dst == nullptr) return dg_set_error("dg_transpose_to_k_major: null pointer");
    if (elem_bytes != 1 && elem_bytes != 2) return dg_set_error("dg_transpose_to_k_major: elem_bytes must be 1 or 2");
    if (batches < 1 || k < 0 || mn < 0 || k_padded < k) return dg_set_error("dg_transpose_to_k_major: bad sizes");
    if (src_ld < mn || dst_ld < k_padded) return dg_set_error("dg_transpose_to_k_major: leading dimension too small");
    if ((dst_ld * elem_bytes) % 16 || (reinterpret_cast<uintptr_t>(dst) % 16) ||
        (batches > 1 && (dst_batch_stride * elem_bytes) % 16))
        return dg_set_error("dg_transpose_to_k_major: destination rows must be 16-byte aligned");
    if (mn == 0 || k_padded == 0) return DG_OK;
    TransposeParams p;
    p.src = reinterpret_cast<const uint8_t*>(src);
    p.dst = reinterpret_cast<uint8_t*>(dst);
    p.src_bs = src_batch_stride; p.src_ld = src_ld; p.dst_bs = dst_batch_stride; p.dst_ld = dst_ld;
    p.k = k; p.mn = mn; p.k_padded = k_padded;
    const dim3 grid((unsigned)ceil_div(k_padded, 64), (unsigned)ceil_div(mn, 64), (unsigned)batches);
    if (grid.x > 0x7fffffffu || grid.y > 65535u || grid.z > 65535u)
        return dg_set_error("dg_transpose_to_k_major: too many tiles");
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    if (elem_bytes == 1) hipLaunchKernelGGL(transpose_to_k_major_kernel<1>, grid, dim3(256), 0, st, p);
    else hipLaunchKernelGGL(transpose_to_k_major_kernel<2>, grid, dim3(256), 0, st, p);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        dg_set_error(hipGetErrorString(e));
        return DG_ELAUNCH;
    }
    return DG_OK;
}
