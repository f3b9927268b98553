// Scale-factor layout transform (HBM-bound byte work).
//
// Behaviour of the reference's transform_sf kernel
// (deep_gemm/include/deep_gemm/transform_sf.hpp:447-639, host side
// csrc/jit_kernels/transform_sf.hpp:15-105): fp32 power-of-two SF -> UE8M0 exponent byte,
// two K-adjacent bytes per int16 (even block low), MN-major output, each SF row repeated
// gran_mn times, M-grouped psum padding rows zeroed, invalid fp32 SF flagged.
//
// One thread produces one output int16; consecutive threads walk the contiguous MN axis so
// the stores are fully coalesced (and the loads too for MN-major sources).  The MN
// axis is stored with an even leading dimension ld = align(MN, 2) (the GEMM kernel fetches
// SF rows in pairs with 4-byte loads); the padding element of every column is written as 0.
#include "dg_common.hpp"
#include "../../include/deep_gemm_amd.h"

namespace dg {

struct SfParams {
    const uint8_t* src;
    int64_t stride_b, stride_mn, stride_k;   // elements of the source type
    int num_batches, sf_mn, sf_k, mn, ld, k64, k32, gran_mn, gran_k;
    const int* psum;
    int num_groups, alignment;
    int16_t* dst;
    int64_t dst_stride_b;
    int* err;
};

// Is SF index `i` (operand rows / K columns [i*gran, (i+1)*gran)) inside the padding of a psum
// layout, i.e. in [ceil(psum[g] / gran), align(psum[g], alignment) / gran) for the group g whose
// aligned end is the first beyond i*gran?  The M-grouped layout pads MN rows, the K-grouped one K.
__device__ __forceinline__ bool psum_is_padding(const SfParams& p, int i, int gran) {
    const int row = i * gran;
    int lo = 0, hi = p.num_groups;   // first g with align(psum[g]) > row
    while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (align_up(p.psum[mid], p.alignment) > row) hi = mid;
        else lo = mid + 1;
    }
    if (lo == p.num_groups) return false;   // beyond the last group: untouched
    return i >= ceil_div(p.psum[lo], gran);
}

// Is SF row i of an M-grouped operand padding?  num_groups >= 1: the psum layout above; -1: `psum`
// holds the m_indices of the rows (gran_mn 1), a negative index marking a padding row.
__device__ __forceinline__ bool mn_is_padding(const SfParams& p, int i) {
    if (p.psum == nullptr) return false;
    if (p.num_groups < 0) return p.psum[i] < 0;
    return psum_is_padding(p, i, p.gran_mn);
}

// kKGrouped: the psum layout splits K (csrc/apis/layout.hpp:94-111): SF of the K padding between
// groups (fp32 per gran_k column, packed int16 per 64-wide column) becomes 0 and is not validated.
// Grid: x walks the MN axis, y the 64-wide K columns (KPB per workgroup), z the batches, so a
// workgroup's K-column facts (range, K-grouped padding) are uniform and computed once.  With an
// MN-contiguous fp32 source (one SF row per MN index, 16-byte aligned columns: the K-grouped and
// MN-major cases) every thread converts 4 consecutive MN with 16-byte loads and an 8-byte store;
// otherwise one.
constexpr int kSfKPB = 2;   // 64-wide K columns per workgroup

// Source bits of SF column j (fp32) for output column k64 half h, or 0 past the range / padding.
template <bool kKGrouped>
__device__ __forceinline__ bool sf_column_live(const SfParams& p, int k64, int h, int& j) {
    const int blk = 2 * k64 + h;   // 32-wide K block
    j = p.gran_k == 128 ? blk >> 2 : blk;
    return __builtin_amdgcn_readfirstlane(blk < p.k32 && j < p.sf_k && !(kKGrouped && psum_is_padding(p, j, p.gran_k)));
}

template <bool kFloat, bool kKGrouped, bool kVec>
__global__ __launch_bounds__(256) void transform_sf_kernel(const SfParams p) {
    constexpr int V = kVec ? 4 : 1;
    const int mn0 = (blockIdx.x * 256 + threadIdx.x) * V;
    const int b = blockIdx.z;
    if (mn0 >= p.ld) return;
#pragma unroll
    for (int kk = 0; kk < kSfKPB; ++kk) {
        const int k64 = blockIdx.y * kSfKPB + kk;
        if (k64 >= p.k64) break;
        uint16_t out[V];
#pragma unroll
        for (int v = 0; v < V; ++v) out[v] = 0;
        if constexpr (kFloat && kVec) {
            // (gran_mn == 1, stride_mn == 1, no psum on MN: row i = mn)
            const uint32_t* s = reinterpret_cast<const uint32_t*>(p.src) + (int64_t)b * p.stride_b;
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                int j;
                if (!sf_column_live<kKGrouped>(p, k64, h, j)) continue;
                const uint32_t* col = s + (int64_t)j * p.stride_k;
                uint32_t bits[4] = {0, 0, 0, 0};
                if (mn0 + 4 <= p.mn) {
                    const i32x4 w = *reinterpret_cast<const i32x4*>(col + mn0);
                    bits[0] = w[0]; bits[1] = w[1]; bits[2] = w[2]; bits[3] = w[3];
                } else {
                    for (int v = 0; v < 4; ++v)
                        if (mn0 + v < p.mn) bits[v] = col[mn0 + v];
                }
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    if ((bits[v] & 0x807fffffu) != 0 && mn0 + v < p.mn && p.err != nullptr) *p.err = 1;
                    out[v] |= (uint16_t)(((bits[v] >> 23) & 0xffu) << (8 * h));
                }
            }
        } else {
            const int mn = mn0;
            const int i = mn / p.gran_mn;
            const bool mn_pad = !kKGrouped && i < p.sf_mn && mn_is_padding(p, i);
            if (mn < p.mn && i < p.sf_mn && !mn_pad) {
                const int64_t row_off = (int64_t)b * p.stride_b + (int64_t)i * p.stride_mn;
                if constexpr (kFloat) {
                    const uint32_t* s = reinterpret_cast<const uint32_t*>(p.src);
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        int j;
                        if (!sf_column_live<kKGrouped>(p, k64, h, j)) continue;
                        const uint32_t bits = s[row_off + (int64_t)j * p.stride_k];
                        if ((bits & 0x807fffffu) != 0 && p.err != nullptr) *p.err = 1;
                        out[0] |= (uint16_t)(((bits >> 23) & 0xffu) << (8 * h));
                    }
                } else {
                    const uint16_t* s = reinterpret_cast<const uint16_t*>(p.src);
                    const bool live =
                        __builtin_amdgcn_readfirstlane(k64 < p.sf_k && !(kKGrouped && psum_is_padding(p, k64, 64)));
                    if (live) out[0] = s[row_off + (int64_t)k64 * p.stride_k];
                }
            }
        }
        int16_t* d = p.dst + (int64_t)b * p.dst_stride_b + (int64_t)k64 * p.ld + mn0;
        if constexpr (kVec) {
            if (mn0 + 4 <= p.ld) {
                *reinterpret_cast<i32x2*>(d) = i32x2{(int)((uint32_t)out[0] | ((uint32_t)out[1] << 16)),
                                                     (int)((uint32_t)out[2] | ((uint32_t)out[3] << 16))};
            } else {
                for (int v = 0; v < 4 && mn0 + v < p.ld; ++v) d[v] = (int16_t)out[v];
            }
        } else {
            d[0] = (int16_t)out[0];
        }
    }
}

// K-major fp32 sources (one contiguous row of SF per MN index, the reference's usual [MN, K / gran]
// layout): a thread owns one MN index and kSfKPBK 64-wide K columns, reading the row's span of
// them with 16-byte loads (the whole 128-byte line for gran_k = 32) instead of one scattered
// float per output; the stores stay coalesced along MN.
constexpr int kSfKPBK = 16;

template <bool kKGrouped>
__global__ __launch_bounds__(256) void transform_sf_kmajor_kernel(const SfParams p) {
    constexpr int F = 2 * kSfKPBK;             // floats of a block's K span at gran_k = 32
    const int mn = blockIdx.x * 256 + threadIdx.x;
    const int b = blockIdx.z, kbase = blockIdx.y * kSfKPBK;
    if (mn >= p.ld) return;
    const int i = mn / p.gran_mn;
    const bool mn_pad = !kKGrouped && i < p.sf_mn && mn_is_padding(p, i);
    const bool row_ok = mn < p.mn && i < p.sf_mn && !mn_pad;
    const int per = p.gran_k == 128 ? 4 : 1;   // 32-wide K blocks per source float
    const int j0 = 2 * kbase / per;            // first source float of the span
    const int nf = F / per;                    // floats of the span (32 or 8)
    uint32_t f[F];
#pragma unroll
    for (int t = 0; t < F; ++t) f[t] = 0;
    if (row_ok) {
        const uint32_t* row = reinterpret_cast<const uint32_t*>(p.src) + (int64_t)b * p.stride_b + (int64_t)i * p.stride_mn;
        if (j0 + nf <= p.sf_k) {
            // (16-byte aligned: the host checks the row stride, j0 is a multiple of 8)
#pragma unroll
            for (int t = 0; t < F / 4; ++t)
                if (t * 4 < nf) {
                    const i32x4 w = *reinterpret_cast<const i32x4*>(row + j0 + 4 * t);
                    f[4 * t] = w[0]; f[4 * t + 1] = w[1]; f[4 * t + 2] = w[2]; f[4 * t + 3] = w[3];
                }
        } else {
            for (int t = 0; t < nf; ++t)
                if (j0 + t < p.sf_k) f[t] = row[j0 + t];
        }
    }
#pragma unroll
    for (int kk = 0; kk < kSfKPBK; ++kk) {
        const int k64 = kbase + kk;
        if (k64 >= p.k64) break;
        uint16_t out = 0;
        if (row_ok) {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                int j;
                if (!sf_column_live<kKGrouped>(p, k64, h, j)) continue;
                // (constant register indices: j - j0 is 2 kk + h, or its quarter at gran_k = 128)
                const uint32_t bits = per == 1 ? f[2 * kk + h] : f[(2 * kk + h) >> 2];
                if ((bits & 0x807fffffu) != 0 && p.err != nullptr) *p.err = 1;
                out |= (uint16_t)(((bits >> 23) & 0xffu) << (8 * h));
            }
        }
        p.dst[(int64_t)b * p.dst_stride_b + (int64_t)k64 * p.ld + mn] = (int16_t)out;
    }
}

}  // namespace dg

extern "C" __attribute__((visibility("hidden"))) int dg_set_error(const char* msg);
namespace dg {
uint32_t* status_words();
}

static int transform_sf_impl(bool k_grouped, const void* src, int32_t src_kind, int64_t stride_b, int64_t stride_mn,
                             int64_t stride_k, int32_t num_batches, int32_t sf_mn, int32_t sf_k,
                             int32_t mn, int32_t k, int32_t gran_mn, int32_t gran_k,
                             const int32_t* psum, int32_t num_groups, int32_t alignment,
                             int16_t* dst, int64_t dst_stride_b, int32_t* err_flag, void* stream) {
    using namespace dg;
    if (src == nullptr || dst == nullptr) return dg_set_error("dg_transform_sf: null pointer");
    if (num_batches < 1 || mn < 0 || k < 0 || sf_mn < 0 || sf_k < 0)
        return dg_set_error("dg_transform_sf: negative size");
    if (gran_mn < 1 || gran_mn > 128 || (gran_mn & (gran_mn - 1)) != 0)
        return dg_set_error("gran_mn only support a power of two in [1, 128]");
    if (src_kind == DG_SF_F32) {
        if (gran_k != 32 && gran_k != 128) return dg_set_error("gran_k must be 32 or 128 for fp32 SF");
        if (sf_k != ceil_div(k, gran_k)) return dg_set_error("dg_transform_sf: sf_k != ceil(K / gran_k)");
    } else if (src_kind == DG_SF_I16) {
        if (gran_k != 32) return dg_set_error("gran_k must be 32");
        if (sf_k != ceil_div(k, 64)) return dg_set_error("dg_transform_sf: sf_k != ceil(K / 64)");
    } else {
        return dg_set_error("dg_transform_sf: unknown src_kind");
    }
    if (sf_mn != ceil_div(mn, gran_mn)) return dg_set_error("dg_transform_sf: sf_mn != ceil(MN / gran_mn)");
    if (num_batches > 1 && dst_stride_b < (int64_t)ceil_div(k, 64) * align_up(mn, 2))
        return dg_set_error("dg_transform_sf: dst batch stride smaller than ceil(K / 64) * align(MN, 2)");
    if (!k_grouped && psum != nullptr && num_groups == -1 && (gran_mn != 1 || num_batches != 1))
        return dg_set_error("dg_transform_sf: an m_indices layout needs gran_mn == 1 and one batch");
    if (!k_grouped && psum != nullptr && num_groups != -1 && (num_groups < 1 || alignment < 1 || alignment % gran_mn != 0))
        return dg_set_error("dg_transform_sf: psum needs num_groups >= 1 and alignment % gran_mn == 0");
    if (k_grouped && (psum == nullptr || num_groups < 1 || num_batches != 1 || alignment < 64 || alignment % 64 != 0))
        return dg_set_error("dg_transform_k_grouped_sf: needs a psum layout, one batch and alignment % 64 == 0");
    SfParams p;
    p.src = reinterpret_cast<const uint8_t*>(src);
    p.stride_b = stride_b; p.stride_mn = stride_mn; p.stride_k = stride_k;
    p.num_batches = num_batches; p.sf_mn = sf_mn; p.sf_k = sf_k; p.mn = mn; p.ld = align_up(mn, 2);
    p.k64 = ceil_div(k, 64); p.k32 = ceil_div(k, 32); p.gran_mn = gran_mn; p.gran_k = gran_k;
    p.psum = psum; p.num_groups = num_groups; p.alignment = alignment;
    p.dst = dst; p.dst_stride_b = dst_stride_b;
    // (without a caller's flag, invalid SFs set the library's sticky error word, which the host
    // API reads at its next call)
    p.err = err_flag != nullptr ? err_flag : reinterpret_cast<int32_t*>(dg::status_words());
    if ((int64_t)p.k64 * p.ld * num_batches == 0) return DG_OK;
    if (ceil_div(p.k64, 2) > 65535 || num_batches > 65535)
        return dg_set_error("dg_transform_sf: K or batch count too large");
    // vector path: fp32 rows one per MN index, MN contiguous, 16-byte aligned columns and batches,
    // no MN padding search, and output rows of a multiple of 4 elements (8-byte stores)
    const bool vec = src_kind == DG_SF_F32 && gran_mn == 1 && stride_mn == 1 && (k_grouped || psum == nullptr) &&
                     (reinterpret_cast<uintptr_t>(src) % 16) == 0 && stride_k % 4 == 0 &&
                     (num_batches == 1 || stride_b % 4 == 0) && p.ld % 4 == 0 &&
                     (reinterpret_cast<uintptr_t>(dst) % 8) == 0 && (num_batches == 1 || dst_stride_b % 4 == 0);
    // K-major path: fp32 rows contiguous along K, 16-byte aligned rows
    const bool kmajor = !vec && src_kind == DG_SF_F32 && stride_k == 1 && (reinterpret_cast<uintptr_t>(src) % 16) == 0 &&
                        stride_mn % 4 == 0 && (num_batches == 1 || stride_b % 4 == 0);
    const dim3 blocks((unsigned)ceil_div(p.ld, 256 * (vec ? 4 : 1)), (unsigned)ceil_div(p.k64, kmajor ? kSfKPBK : kSfKPB),
                      (unsigned)num_batches);
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    if (kmajor) {
        if (k_grouped) hipLaunchKernelGGL((transform_sf_kmajor_kernel<true>), blocks, dim3(256), 0, st, p);
        else hipLaunchKernelGGL((transform_sf_kmajor_kernel<false>), blocks, dim3(256), 0, st, p);
    } else if (vec) {
        if (k_grouped) hipLaunchKernelGGL((transform_sf_kernel<true, true, true>), blocks, dim3(256), 0, st, p);
        else hipLaunchKernelGGL((transform_sf_kernel<true, false, true>), blocks, dim3(256), 0, st, p);
    } else if (k_grouped) {
        if (src_kind == DG_SF_F32)
            hipLaunchKernelGGL((transform_sf_kernel<true, true, false>), blocks, dim3(256), 0, st, p);
        else
            hipLaunchKernelGGL((transform_sf_kernel<false, true, false>), blocks, dim3(256), 0, st, p);
    } else {
        if (src_kind == DG_SF_F32)
            hipLaunchKernelGGL((transform_sf_kernel<true, false, false>), blocks, dim3(256), 0, st, p);
        else
            hipLaunchKernelGGL((transform_sf_kernel<false, false, false>), blocks, dim3(256), 0, st, p);
    }
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        dg_set_error(hipGetErrorString(e));
        return DG_ELAUNCH;
    }
    return DG_OK;
}

extern "C" int dg_transform_sf(const void* src, int32_t src_kind, int64_t stride_b, int64_t stride_mn,
                               int64_t stride_k, int32_t num_batches, int32_t sf_mn, int32_t sf_k,
                               int32_t mn, int32_t k, int32_t gran_mn, int32_t gran_k,
                               const int32_t* psum, int32_t num_groups, int32_t alignment,
                               int16_t* dst, int64_t dst_stride_b, int32_t* err_flag, void* stream) {
    return transform_sf_impl(false, src, src_kind, stride_b, stride_mn, stride_k, num_batches, sf_mn, sf_k, mn, k,
                             gran_mn, gran_k, psum, num_groups, alignment, dst, dst_stride_b, err_flag, stream);
}

extern "C" int dg_transform_k_grouped_sf(const void* src, int32_t src_kind, int64_t stride_mn, int64_t stride_k,
                                         int32_t sf_mn, int32_t sf_k, int32_t mn, int32_t k, int32_t gran_mn,
                                         int32_t gran_k, const int32_t* psum, int32_t num_groups, int32_t alignment,
                                         int16_t* dst, int32_t* err_flag, void* stream) {
    return transform_sf_impl(true, src, src_kind, 0, stride_mn, stride_k, 1, sf_mn, sf_k, mn, k, gran_mn, gran_k,
                             psum, num_groups, alignment, dst, 0, err_flag, stream);
}
