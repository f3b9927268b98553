// MN-major -> K-major operand copy (HBM-bound byte work).
//
// The GEMM kernels stream K-major operand rows; an operand the caller holds MN-major (the `tn`
// / `nn` / `tt` layouts, the K-grouped wgrad operands [Ktot, M], einsum views whose contraction
// axis is not the innermost) is transposed once on the device.  One workgroup moves a tile of
// 128 / E K-indices x 128 bytes of MN (16 KB for e4m3, 8 KB for bf16) through LDS: every
// thread keeps its loads of the tile in flight at once, transposes 4-byte blocks in registers
// (v_perm_b32) into K-contiguous words, and both the loads (rows of MN) and the stores (rows of
// K) move whole 128-byte lines per group of 8 threads.  Columns K .. k_padded-1 of the output are written as zeros so the
// result is directly a 16-byte-aligned K-major operand.
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
    constexpr int ROWB = 128;             // bytes of a tile row (MN) and of an output segment (K)
    constexpr int TM = ROWB / E;          // MN elements of a tile
    constexpr int TK = ROWB / E;          // K elements of a tile
    constexpr int VEC = 16 / E;           // elements per 16-byte access
    constexpr int KP = 4 / E;             // K elements of one 32-bit word
    constexpr int PASS = 256 / 8;         // rows per pass (8 threads per 128-byte row)
    constexpr int NSTORE = TM / PASS;     // stores per thread
    static_assert(TK / KP == PASS, "one K word per thread group");
    // Transposed tile: row = MN index, ROWB bytes of K in 16-byte chunks, chunk j of row r stored
    // at j ^ ((r / 16) % 8): a wave's word writes (its lanes 16 rows apart) then spread over the
    // banks, and every 16-byte read stays aligned.
    __shared__ __align__(16) uint8_t tile_t[TM][ROWB];
    auto chunk_at = [](int r, int j) { return ((j ^ ((r >> 4) & 7)) << 4); };

    const int tid = threadIdx.x;
    const int k0 = blockIdx.x * TK, mn0 = blockIdx.y * TM, b = blockIdx.z;
    const uint8_t* src = p.src + ((int64_t)b * p.src_bs) * E;
    uint8_t* dst = p.dst + ((int64_t)b * p.dst_bs) * E;
    const int g = tid / 8;                // K word of the tile: K rows [KP g, KP g + KP)
    const int c = (tid % 8) * VEC;        // MN elements [c, c + VEC) of the tile

    // load: KP source rows (K indices) of 16 MN bytes each, all in flight at once
    const bool vec_ok = (p.src_ld % VEC) == 0 && (reinterpret_cast<uintptr_t>(src) % 16) == 0;
    i32x4 w[KP];
#pragma unroll
    for (int i = 0; i < KP; ++i) {
        const int k = k0 + KP * g + i, mn = mn0 + c;
        w[i] = i32x4{0, 0, 0, 0};
        if (k < p.k) {
            const uint8_t* s = src + ((int64_t)k * p.src_ld + mn) * E;
            if (vec_ok && mn + VEC <= p.mn) {
                w[i] = *reinterpret_cast<const i32x4*>(s);
            } else {
                uint8_t* wb = reinterpret_cast<uint8_t*>(&w[i]);
                for (int j = 0; j < VEC; ++j)
                    if (mn + j < p.mn)
                        for (int e = 0; e < E; ++e) wb[j * E + e] = s[j * E + e];
            }
        }
    }
    // Transpose in registers: for each of the VEC MN elements, one 32-bit word holding its KP
    // K-consecutive values (v_perm_b32 picks bytes from a pair of words: selector byte n takes
    // byte n of the second operand for n < 4, byte n - 4 of the first for n >= 4).
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        uint32_t t[4];
        if constexpr (E == 1) {
            // 4x4 byte block: rows = K 0..3 (words w[i][q]), columns = MN 4q .. 4q + 3
            const uint32_t r0 = w[0][q], r1 = w[1][q], r2 = w[2][q], r3 = w[3][q];
            const uint32_t lo01 = __builtin_amdgcn_perm(r1, r0, 0x05010400u);   // r0.b0 r1.b0 r0.b1 r1.b1
            const uint32_t hi01 = __builtin_amdgcn_perm(r1, r0, 0x07030602u);   // r0.b2 r1.b2 r0.b3 r1.b3
            const uint32_t lo23 = __builtin_amdgcn_perm(r3, r2, 0x05010400u);
            const uint32_t hi23 = __builtin_amdgcn_perm(r3, r2, 0x07030602u);
            t[0] = __builtin_amdgcn_perm(lo23, lo01, 0x05040100u);   // MN 4q:     K 0..3
            t[1] = __builtin_amdgcn_perm(lo23, lo01, 0x07060302u);   // MN 4q + 1
            t[2] = __builtin_amdgcn_perm(hi23, hi01, 0x05040100u);   // MN 4q + 2
            t[3] = __builtin_amdgcn_perm(hi23, hi01, 0x07060302u);   // MN 4q + 3
#pragma unroll
            for (int j = 0; j < 4; ++j)
                *reinterpret_cast<uint32_t*>(&tile_t[c + 4 * q + j][chunk_at(c + 4 * q + j, g >> 2) + (g & 3) * 4]) = t[j];
        } else {
            // 2x2 block of 16-bit elements: rows = K 0..1, columns = MN 2q, 2q + 1
            const uint32_t r0 = w[0][q], r1 = w[1][q];
            t[0] = __builtin_amdgcn_perm(r1, r0, 0x05040100u);   // MN 2q:     K 0, 1
            t[1] = __builtin_amdgcn_perm(r1, r0, 0x07060302u);   // MN 2q + 1
#pragma unroll
            for (int j = 0; j < 2; ++j)
                *reinterpret_cast<uint32_t*>(&tile_t[c + 2 * q + j][chunk_at(c + 2 * q + j, g >> 2) + (g & 3) * 4]) = t[j];
        }
    }
    __syncthreads();

    // store: output row = MN index, 128 bytes of K from 8 threads (whole lines per instruction),
    // each thread's 16 bytes one LDS read of the transposed tile
#pragma unroll
    for (int i = 0; i < NSTORE; ++i) {
        const int r = i * PASS + tid / 8;     // MN within the tile
        const int cb = (tid % 8) * 16;        // byte of the tile's K segment
        const int mn = mn0 + r, k = k0 + cb / E;
        if (mn >= p.mn || k >= p.k_padded) continue;
        const i32x4 o = *reinterpret_cast<const i32x4*>(&tile_t[r][chunk_at(r, tid % 8)]);
        uint8_t* d = dst + ((int64_t)mn * p.dst_ld + k) * E;
        if (k + VEC <= p.k_padded) {
            *reinterpret_cast<i32x4*>(d) = o;
        } else {
            const uint8_t* ob = reinterpret_cast<const uint8_t*>(&o);
            for (int j = 0; j < VEC && k + j < p.k_padded; ++j)
                for (int e = 0; e < E; ++e) d[j * E + e] = ob[j * E + e];
        }
    }
}


// FP4 (e2m1) operand packed along MN -> packed along K.  Source byte (b, k, j) holds MN 2j (low
// nibble) and 2j + 1 (high nibble) of K row k; output byte (b, mn, j) holds K 2j (low) and 2j + 1
// (high) of MN row mn, zero past k.  One workgroup moves 64 K x 128 MN: it loads 64 source rows
// of 64 bytes (16 bytes a thread, one coalesced line per 4 threads) into LDS, then each thread
// gathers the 32 nibble pairs of 16 output bytes of one MN row and stores them at once.
struct Fp4RepackParams {
    const uint8_t* src;
    uint8_t* dst;
    int64_t src_bs, src_ld, dst_bs, dst_ld;   // bytes
    int k, mn, k_padded;                      // elements
};

__global__ __launch_bounds__(256) void fp4_repack_k_major_kernel(const Fp4RepackParams p) {
    constexpr int TK = 64, TMN = 128, PITCH = TMN / 2 + 4;   // (+4: rows 16 lanes apart on other banks)
    __shared__ __align__(16) uint8_t tile[TK][PITCH];
    const int tid = threadIdx.x;
    const int k0 = blockIdx.x * TK, mn0 = blockIdx.y * TMN, b = blockIdx.z;
    const uint8_t* src = p.src + (int64_t)b * p.src_bs;
    uint8_t* dst = p.dst + (int64_t)b * p.dst_bs;
    const int mnb = (p.mn + 1) / 2;                            // source bytes of a K row
    {
        const int kr = tid / 4, cb = (tid % 4) * 16;           // K row of the tile, byte of its row
        const int k = k0 + kr, j = mn0 / 2 + cb;
        i32x4 w = {0, 0, 0, 0};
        if (k < p.k) {
            const uint8_t* s = src + (int64_t)k * p.src_ld + j;
            if (j + 16 <= mnb && (reinterpret_cast<uintptr_t>(s) % 16) == 0) {
                w = *reinterpret_cast<const i32x4*>(s);
            } else {
                uint8_t* wb = reinterpret_cast<uint8_t*>(&w);
                for (int e = 0; e < 16; ++e)
                    if (j + e < mnb) wb[e] = s[e];
            }
        }
        *reinterpret_cast<i32x4*>(&tile[kr][cb]) = w;   // (PITCH keeps 16-byte alignment: 68 = 4 x 17)
    }
    __syncthreads();
    const int r = tid / 2, half = tid % 2;                     // MN row of the tile, 32-K half
    const int mn = mn0 + r, kb = k0 / 2 + half * 16;           // output byte of the row
    if (mn >= p.mn || 2 * kb >= p.k_padded) return;
    const int sh = (r & 1) * 4;
    i32x4 o;
    uint8_t* ob = reinterpret_cast<uint8_t*>(&o);
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        const int kk = half * 32 + 2 * j;                      // K of the tile (rows past k hold zeros)
        const uint32_t lo = (tile[kk][r / 2] >> sh) & 15u, hi = (tile[kk + 1][r / 2] >> sh) & 15u;
        ob[j] = (uint8_t)(lo | (hi << 4));
    }
    uint8_t* d = dst + (int64_t)mn * p.dst_ld + kb;
    if (2 * kb + 32 <= p.k_padded) {
        *reinterpret_cast<i32x4*>(d) = o;
    } else {
        for (int j = 0; 2 * (kb + j) < p.k_padded; ++j) d[j] = ob[j];
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
    const int tile = 128 / elem_bytes;   // K and MN elements of a workgroup's tile
    const dim3 grid((unsigned)ceil_div(k_padded, tile), (unsigned)ceil_div(mn, tile), (unsigned)batches);
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

extern "C" int dg_fp4_to_k_major(const void* src, int32_t batches, int64_t src_batch_stride, int64_t src_ld, int32_t k,
                                 int32_t mn, void* dst, int64_t dst_batch_stride, int64_t dst_ld, int32_t k_padded,
                                 void* stream) {
    using namespace dg;
    if (src == nullptr || dst == nullptr) return dg_set_error("dg_fp4_to_k_major: null pointer");
    if (batches < 1 || k < 0 || mn < 0 || k_padded < k || k_padded % 2)
        return dg_set_error("dg_fp4_to_k_major: bad sizes");
    if (src_ld < (mn + 1) / 2 || dst_ld * 2 < k_padded)
        return dg_set_error("dg_fp4_to_k_major: leading dimension too small");
    if (dst_ld % 16 || (reinterpret_cast<uintptr_t>(dst) % 16) || (batches > 1 && dst_batch_stride % 16))
        return dg_set_error("dg_fp4_to_k_major: destination rows must be 16-byte aligned");
    if (mn == 0 || k_padded == 0) return DG_OK;
    Fp4RepackParams p;
    p.src = reinterpret_cast<const uint8_t*>(src);
    p.dst = reinterpret_cast<uint8_t*>(dst);
    p.src_bs = src_batch_stride; p.src_ld = src_ld; p.dst_bs = dst_batch_stride; p.dst_ld = dst_ld;
    p.k = k; p.mn = mn; p.k_padded = k_padded;
    const dim3 grid((unsigned)ceil_div(k_padded, 64), (unsigned)ceil_div(mn, 128), (unsigned)batches);
    if (grid.y > 65535u || grid.z > 65535u) return dg_set_error("dg_fp4_to_k_major: too many tiles");
    hipLaunchKernelGGL(fp4_repack_k_major_kernel, grid, dim3(256), 0, reinterpret_cast<hipStream_t>(stream), p);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        dg_set_error(hipGetErrorString(e));
        return DG_ELAUNCH;
    }
    return DG_OK;
}
