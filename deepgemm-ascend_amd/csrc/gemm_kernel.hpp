// Block-scaled GEMM kernel for gfx950 (MI355X).
//
// D = alpha * A . B^T (+ bias | + D) for K-major A [M,K] and B [N,K], with one UE8M0 scale
// per 32 K-elements and per row of each operand (the MX recipe of the reference's
// fp8_gemm_impl, deep_gemm/include/deep_gemm/fp8_gemm.hpp:36-287), computed on CDNA4
// v_mfma_scale_f32_16x16x128_f8f6f4 (e4m3 / e2m1 operands) or v_mfma_f32_16x16x32_bf16.
//
// Data flow of one 256-thread workgroup (4 waves, 2 x 2 over the BM x BN tile):
//   HBM/L2 --buffer_load_dwordx4 ... lds--> LDS stage (double buffered, XOR-swizzled
//   16-byte slots) --ds_read_b128--> VGPR fragments --MFMA--> fp32 accumulators
//   --epilogue (alpha / bias / accumulate, RNE bf16 cast) in registers--> D.
// Scales stream beside the data: two packed int16 rows of the required SF layout per
// 128-K chunk are loaded into VGPRs one chunk ahead, re-laid out in LDS so that each lane
// fetches the bytes of all its row blocks with one ds_read_b64, and fed to the MFMA as the
// per-lane scale operand (byte picked with op_sel).
//
// MFMA register layouts (measured on gfx950):
//   16x16x128 e4m3 operand, lane l = r + 16 q (r = row, q = lane group):
//       bytes [0,16) hold K [16q, 16q+16), bytes [16,32) hold K [64+16q, 64+16q+16)
//   16x16x128 e2m1 operand: 16 bytes hold K [32q, 32q+32) (low nibble = even k)
//   scale operand of lane (r, q): UE8M0 exponent of K-block q (K [32q, 32q+32)) of row r
//   16x16x32 bf16 operand: 8 values hold K [8q, 8q+8)
//   accumulator: lane l, element i -> (row 4*(l/16) + i of the MFMA "A" side, column l%16)
// The kernel feeds B (n) as the MFMA "A" operand and A (m) as the "B" operand, so each lane
// ends with four consecutive n of one output row m: 8-byte (bf16) / 16-byte (fp32) stores.
#pragma once

#include <utility>
#include "dg_common.hpp"

namespace dg {

struct KParams {
    const uint8_t* a;
    const uint8_t* b;
    uint8_t* d;
    const uint16_t* sfa;
    const uint16_t* sfb;
    const uint8_t* bias;
    const int* layout;
    int m, n, k, num_groups;
    int64_t lda, ldb;          // bytes
    int64_t ldd;               // elements of D
    int64_t bsa, bsb;          // bytes
    int64_t bsd;               // elements of D
    int64_t sfa_ld, sfb_ld, sfa_bs, sfb_bs;   // int16 elements
    int gemm_type, out_f32, accumulate, has_bias, alignment, vec_store;
    float alpha;
    int num_m_blocks, num_n_blocks;
    int kbytes_a, kbytes_b;    // bytes of one K row (multiple of 16)
    int group_m;               // tile-order swizzle width along M
};

template <int N>
struct Int { static constexpr int value = N; };

template <typename F, int... Is>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, Is...>) {
    (f(Int<Is>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
    static_for_impl(f, std::make_integer_sequence<int, N>{});
}

// Slot swizzle inside one LDS row: 8 slots (128-byte rows) or 4 slots (64-byte rows).
template <int SPR>
__device__ __forceinline__ int slot_swizzle(int row) {
    if constexpr (SPR == 8) return row & 7;
    else return (row >> 1) & 3;
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, int64_t bytes) {
    if (bytes > 0x7fffffffLL) bytes = 0x7fffffffLL;
    if (bytes < 0) bytes = 0;
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                             (int)kBufferRsrcWord3);
}

// Spread consecutive workgroup ids over the 8 XCDs so that each XCD (own L2) receives a
// contiguous range of tiles; hardware dispatches workgroup i to XCD i % 8.
__device__ __forceinline__ int xcd_remap(int bid, int nblocks) {
    constexpr int kXCD = 8;
    const int per = nblocks / kXCD;
    if (bid >= per * kXCD) return bid;
    return (bid % kXCD) * per + bid / kXCD;
}

// GROUP_M tile order: walk n inside bands of `gm` m-blocks (L2 reuse of A and B tiles).
__device__ __forceinline__ void swizzle_tile(int t, int nm, int nn, int gm, int& mb, int& nb) {
    const int band = gm * nn;
    const int first_m = (t / band) * gm;
    const int size = min(nm - first_m, gm);
    const int in_band = t % band;
    mb = first_m + in_band % size;
    nb = in_band / size;
}

template <int FMT_A, int FMT_B, int OPSEL_A, int OPSEL_B>
__device__ __forceinline__ f32x4 mfma_scaled(const i32x8& a, const i32x8& b, const f32x4& c,
                                             int sa, int sb) {
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, FMT_A, FMT_B, OPSEL_A, sa,
                                                            OPSEL_B, sb);
}

template <int BM, int BN, int KIND>
__global__ __launch_bounds__(256, 1) void gemm_kernel(const KParams p) {
    constexpr bool kAFp4 = KIND == kFP4FP4;
    constexpr bool kBFp4 = KIND == kFP8FP4 || KIND == kFP4FP4;
    constexpr bool kBf16 = KIND == kBF16;
    constexpr int kFmtA = kAFp4 ? kFmtE2M1 : kFmtE4M3;
    constexpr int kFmtB = kBFp4 ? kFmtE2M1 : kFmtE4M3;
    constexpr int RBA = kAFp4 ? 64 : 128;       // bytes of one row per K chunk
    constexpr int RBB = kBFp4 ? 64 : 128;
    constexpr int SPRA = RBA / 16, SPRB = RBB / 16;
    constexpr int WM = BM / 2, WN = BN / 2;      // wave tile
    constexpr int TM = WM / 16, TN = WN / 16;    // MFMA blocks per wave
    static_assert(TM >= 1 && TM <= 8 && TN >= 1 && TN <= 8, "wave tile must be 16..128");
    constexpr int A_BYTES = BM * RBA, B_BYTES = BN * RBB;
    static_assert(A_BYTES % 1024 == 0 && B_BYTES % 1024 == 0, "tile rows must fill waves");
    constexpr int SC_BYTES = kBf16 ? 0 : 1024;
    constexpr int STAGE = A_BYTES + B_BYTES + 2 * SC_BYTES;
    __shared__ __attribute__((aligned(1024))) uint8_t smem[2 * STAGE];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave & 1, wn = wave >> 1;
    const int r = lane & 15, q = lane >> 4;

    // ------------------------------------------------------------------ tile selection
    const int nm = p.num_m_blocks, nn = p.num_n_blocks;
    int t = xcd_remap(blockIdx.x, gridDim.x);
    int batch = 0;
    if (p.gemm_type == kBatched || p.gemm_type == kMasked) {
        batch = t / (nm * nn);
        t -= batch * nm * nn;
    }
    int mb, nb;
    swizzle_tile(t, nm, nn, p.group_m, mb, nb);
    const int m0 = mb * BM, n0 = nb * BN;
    const int M = p.m, N = p.n;

    const uint8_t* a_base = p.a;
    const uint8_t* b_base = p.b;
    const uint16_t* sfa = p.sfa;
    const uint16_t* sfb = p.sfb;
    uint8_t* d_base = p.d;
    const int out_esize = p.out_f32 ? 4 : 2;
    int group = 0;          // B operand group
    int valid_end = M;      // rows >= valid_end are padding (psum) / not written (masked)
    bool zero_tile = false;

    if (p.gemm_type == kBatched || p.gemm_type == kMasked) {
        group = batch;
        a_base += (int64_t)batch * p.bsa;
        d_base += (int64_t)batch * p.bsd * out_esize;
        if (!kBf16) sfa += (int64_t)batch * p.sfa_bs;
        if (p.gemm_type == kMasked) {
            valid_end = min(M, p.layout[batch]);
            if (m0 >= valid_end) return;   // whole tile beyond masked_m: nothing to write
        }
    } else if (p.gemm_type == kMGroupedPsum) {
        int found = -1;
        for (int base = 0; base < p.num_groups; base += 64) {
            const int gi = base + lane;
            bool pred = false;
            if (gi < p.num_groups) pred = align_up(p.layout[gi], p.alignment) > m0;
            const uint64_t mask = __ballot(pred);
            if (mask) { found = base + __builtin_ctzll(mask); break; }
        }
        if (found < 0) {
            zero_tile = true;
        } else {
            group = found;
            valid_end = min(M, p.layout[found]);
            if (valid_end <= m0) zero_tile = true;
        }
    } else if (p.gemm_type == kMGroupedIdx) {
        group = p.layout[m0];
        if (group < 0) zero_tile = true;
    }

    if (zero_tile) {
        // Padding-only tile of an M-grouped layout: its D rows are exact zeros.
        const int rows = min(BM, M - m0), cols = min(BN, N - n0);
        for (int e = tid; e < rows * cols; e += 256) {
            const int rr = e / cols, cc = e % cols;
            const int64_t off = (int64_t)(m0 + rr) * p.ldd + n0 + cc;
            if (p.out_f32) reinterpret_cast<float*>(d_base)[off] = 0.f;
            else reinterpret_cast<uint16_t*>(d_base)[off] = 0;
        }
        return;
    }
    if (p.gemm_type == kMGroupedPsum || p.gemm_type == kMGroupedIdx || p.gemm_type == kBatched ||
        p.gemm_type == kMasked) {
        b_base += (int64_t)group * p.bsb;
        if (!kBf16) sfb += (int64_t)group * p.sfb_bs;
    }

    const int rows_a = min(BM, M - m0);
    const int rows_b = min(BN, N - n0);
    const int64_t lda = p.lda, ldb = p.ldb;
    const __amdgpu_buffer_rsrc_t rs_a = make_rsrc(a_base + (int64_t)m0 * lda, (int64_t)rows_a * lda);
    const __amdgpu_buffer_rsrc_t rs_b = make_rsrc(b_base + (int64_t)n0 * ldb, (int64_t)rows_b * ldb);
    const int kbytes_a = p.kbytes_a, kbytes_b = p.kbytes_b;
    const int KC = kBf16 ? 64 : 128;
    const int num_chunks = ceil_div(p.k, KC);
    const int nk64 = ceil_div(p.k, 64);

    // ------------------------------------------------------------------ loaders
    auto issue_data = [&](int c, int s) {
        uint8_t* sA = smem + s * STAGE;
        uint8_t* sB = sA + A_BYTES;
        const int kb_a = c * RBA, kb_b = c * RBB;
#pragma unroll
        for (int it = 0; it < A_BYTES / 4096 + (A_BYTES % 4096 ? 1 : 0); ++it) {
            if (A_BYTES % 4096 == 0 || (it * 256 + wave * 64) * 16 < A_BYTES) {
                const int slot = it * 256 + tid;
                const int row = slot / SPRA;
                const int logical = (slot % SPRA) ^ slot_swizzle<SPRA>(row);
                const int kb = kb_a + logical * 16;
                const uint32_t voff = (row < rows_a && kb < kbytes_a)
                                          ? (uint32_t)(row * lda + kb) : kOOBOffset;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    rs_a, (lds_void*)(sA + (it * 256 + wave * 64) * 16), 16, voff, 0, 0, 0);
            }
        }
#pragma unroll
        for (int it = 0; it < B_BYTES / 4096 + (B_BYTES % 4096 ? 1 : 0); ++it) {
            if (B_BYTES % 4096 == 0 || (it * 256 + wave * 64) * 16 < B_BYTES) {
                const int slot = it * 256 + tid;
                const int row = slot / SPRB;
                const int logical = (slot % SPRB) ^ slot_swizzle<SPRB>(row);
                const int kb = kb_b + logical * 16;
                const uint32_t voff = (row < rows_b && kb < kbytes_b)
                                          ? (uint32_t)(row * ldb + kb) : kOOBOffset;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    rs_b, (lds_void*)(sB + (it * 256 + wave * 64) * 16), 16, voff, 0, 0, 0);
            }
        }
    };

    constexpr int NSA = (2 * BM + 255) / 256, NSB = (2 * BN + 255) / 256;
    uint32_t sa_reg[NSA], sb_reg[NSB];
    auto issue_scales = [&](int c) {
        if constexpr (!kBf16) {
#pragma unroll
            for (int i = 0; i < NSA; ++i) {
                const int idx = i * 256 + tid;
                const int h = idx / BM, row = idx % BM, k64 = 2 * c + h;
                sa_reg[i] = (idx < 2 * BM && row < rows_a && k64 < nk64)
                                ? (uint32_t)sfa[(int64_t)k64 * p.sfa_ld + m0 + row] : 0x7f7fu;
            }
#pragma unroll
            for (int i = 0; i < NSB; ++i) {
                const int idx = i * 256 + tid;
                const int h = idx / BN, row = idx % BN, k64 = 2 * c + h;
                sb_reg[i] = (idx < 2 * BN && row < rows_b && k64 < nk64)
                                ? (uint32_t)sfb[(int64_t)k64 * p.sfb_ld + n0 + row] : 0x7f7fu;
            }
        }
    };
    // LDS scale layout per operand: byte (q*16 + r)*16 + w*8 + jj holds the exponent of K-block
    // q of tile row (w*T + jj)*16 + r, T = row blocks per wave; lane (r, q) of wave w reads its
    // T bytes with one 8-byte load.
    auto write_scales = [&](int s) {
        if constexpr (!kBf16) {
            uint8_t* sSA = smem + s * STAGE + A_BYTES + B_BYTES;
            uint8_t* sSB = sSA + SC_BYTES;
#pragma unroll
            for (int i = 0; i < NSA; ++i) {
                const int idx = i * 256 + tid;
                if (idx < 2 * BM) {
                    const int h = idx / BM, row = idx % BM;
                    const int j = row >> 4, rr = row & 15;
                    const int pos = ((2 * h) * 16 + rr) * 16 + (j / TM) * 8 + (j % TM);
                    sSA[pos] = (uint8_t)(sa_reg[i] & 0xff);
                    sSA[pos + 256] = (uint8_t)(sa_reg[i] >> 8);
                }
            }
#pragma unroll
            for (int i = 0; i < NSB; ++i) {
                const int idx = i * 256 + tid;
                if (idx < 2 * BN) {
                    const int h = idx / BN, row = idx % BN;
                    const int j = row >> 4, rr = row & 15;
                    const int pos = ((2 * h) * 16 + rr) * 16 + (j / TN) * 8 + (j % TN);
                    sSB[pos] = (uint8_t)(sb_reg[i] & 0xff);
                    sSB[pos + 256] = (uint8_t)(sb_reg[i] >> 8);
                }
            }
        }
    };

    f32x4 acc[TN][TM];
#pragma unroll
    for (int i = 0; i < TN; ++i)
#pragma unroll
        for (int j = 0; j < TM; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    auto load_frag = [&](const uint8_t* base, int R, auto spr_tag) -> i32x8 {
        constexpr int SPR = decltype(spr_tag)::value;
        i32x8 f;
        if constexpr (SPR == 8) {
            const int sw = slot_swizzle<8>(R);
            const i32x4 lo = *reinterpret_cast<const i32x4*>(base + R * 128 + ((q ^ sw) << 4));
            const i32x4 hi = *reinterpret_cast<const i32x4*>(base + R * 128 + (((q + 4) ^ sw) << 4));
            f = i32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        } else {
            const int sw = slot_swizzle<4>(R);
            const i32x4 lo = *reinterpret_cast<const i32x4*>(base + R * 64 + ((q ^ sw) << 4));
            f = i32x8{lo[0], lo[1], lo[2], lo[3], 0, 0, 0, 0};
        }
        return f;
    };

    auto compute = [&](int s) {
        const uint8_t* sA = smem + s * STAGE;
        const uint8_t* sB = sA + A_BYTES;
        i32x8 fa[TM];
#pragma unroll
        for (int jm = 0; jm < TM; ++jm) fa[jm] = load_frag(sA, wm * WM + jm * 16 + r, Int<SPRA>{});
        if constexpr (kBf16) {
#pragma unroll
            for (int jn = 0; jn < TN; ++jn) {
                const i32x8 fb = load_frag(sB, wn * WN + jn * 16 + r, Int<SPRB>{});
                const i32x4 blo = {fb[0], fb[1], fb[2], fb[3]}, bhi = {fb[4], fb[5], fb[6], fb[7]};
#pragma unroll
                for (int jm = 0; jm < TM; ++jm) {
                    const i32x4 alo = {fa[jm][0], fa[jm][1], fa[jm][2], fa[jm][3]};
                    const i32x4 ahi = {fa[jm][4], fa[jm][5], fa[jm][6], fa[jm][7]};
                    acc[jn][jm] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                        __builtin_bit_cast(bf16x8, blo), __builtin_bit_cast(bf16x8, alo), acc[jn][jm], 0, 0, 0);
                    acc[jn][jm] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                        __builtin_bit_cast(bf16x8, bhi), __builtin_bit_cast(bf16x8, ahi), acc[jn][jm], 0, 0, 0);
                }
            }
        } else {
            const uint8_t* sSA = sA + A_BYTES + B_BYTES;
            const uint8_t* sSB = sSA + SC_BYTES;
            const i32x2 sa2 = *reinterpret_cast<const i32x2*>(sSA + (q * 16 + r) * 16 + wm * 8);
            const i32x2 sb2 = *reinterpret_cast<const i32x2*>(sSB + (q * 16 + r) * 16 + wn * 8);
            static_for<TN>([&](auto jn_c) {
                constexpr int jn = decltype(jn_c)::value;
                const i32x8 fb = load_frag(sB, wn * WN + jn * 16 + r, Int<SPRB>{});
                static_for<TM>([&](auto jm_c) {
                    constexpr int jm = decltype(jm_c)::value;
                    acc[jn][jm] = mfma_scaled<kFmtB, kFmtA, jn % 4, jm % 4>(
                        fb, fa[jm], acc[jn][jm], sb2[jn / 4], sa2[jm / 4]);
                });
            });
        }
    };

    // ------------------------------------------------------------------ main loop
    if (num_chunks > 0) {
        issue_data(0, 0);
        issue_scales(0);
    }
    for (int c = 0; c < num_chunks; ++c) {
        const int s = c & 1;
        __builtin_amdgcn_s_waitcnt(0);   // chunk c data (LDS) and scales (VGPR) have landed
        write_scales(s);
        __syncthreads();
        if (c + 1 < num_chunks) {
            issue_data(c + 1, s ^ 1);
            issue_scales(c + 1);
        }
        compute(s);
    }

    // ------------------------------------------------------------------ epilogue
    const float alpha = p.alpha;
    const bool grouped_rows = p.gemm_type == kMGroupedPsum || p.gemm_type == kMGroupedIdx;
#pragma unroll
    for (int jm = 0; jm < TM; ++jm) {
        const int m = m0 + wm * WM + jm * 16 + r;
        if (m >= M) continue;
        if (p.gemm_type == kMasked && m >= valid_end) continue;
        bool pad_row = false;
        if (p.gemm_type == kMGroupedPsum) pad_row = m >= valid_end;
        else if (p.gemm_type == kMGroupedIdx) pad_row = p.layout[m] != group;
        (void)grouped_rows;
#pragma unroll
        for (int jn = 0; jn < TN; ++jn) {
            const int nbase = n0 + wn * WN + jn * 16 + 4 * q;
            if (nbase >= N) continue;
            float v[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) v[i] = acc[jn][jm][i] * alpha;
            if (pad_row) {
#pragma unroll
                for (int i = 0; i < 4; ++i) v[i] = 0.f;
            } else {
                if (p.has_bias) {
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        if (nbase + i < N)
                            v[i] += p.out_f32 ? reinterpret_cast<const float*>(p.bias)[nbase + i]
                                              : bf16_to_f32(reinterpret_cast<const uint16_t*>(p.bias)[nbase + i]);
                    }
                }
            }
            const int64_t off = (int64_t)m * p.ldd + nbase;
            const bool full = p.vec_store && nbase + 3 < N;
            if (p.out_f32) {
                float* dp = reinterpret_cast<float*>(d_base) + off;
                if (full) {
                    f32x4 o = {v[0], v[1], v[2], v[3]};
                    if (p.accumulate && !pad_row) o += *reinterpret_cast<const f32x4*>(dp);
                    *reinterpret_cast<f32x4*>(dp) = o;
                } else {
                    for (int i = 0; i < 4 && nbase + i < N; ++i)
                        dp[i] = (p.accumulate && !pad_row) ? dp[i] + v[i] : v[i];
                }
            } else {
                uint16_t* dp = reinterpret_cast<uint16_t*>(d_base) + off;
                if (full) {
                    if (p.accumulate && !pad_row) {
                        const i32x2 old = *reinterpret_cast<const i32x2*>(dp);
                        v[0] += bf16_to_f32((uint16_t)(old[0] & 0xffff));
                        v[1] += bf16_to_f32((uint16_t)((uint32_t)old[0] >> 16));
                        v[2] += bf16_to_f32((uint16_t)(old[1] & 0xffff));
                        v[3] += bf16_to_f32((uint16_t)((uint32_t)old[1] >> 16));
                    }
                    i32x2 o;
                    o[0] = (int)((uint32_t)f32_to_bf16_rne(v[0]) | ((uint32_t)f32_to_bf16_rne(v[1]) << 16));
                    o[1] = (int)((uint32_t)f32_to_bf16_rne(v[2]) | ((uint32_t)f32_to_bf16_rne(v[3]) << 16));
                    *reinterpret_cast<i32x2*>(dp) = o;
                } else {
                    for (int i = 0; i < 4 && nbase + i < N; ++i) {
                        float x = v[i];
                        if (p.accumulate && !pad_row) x += bf16_to_f32(dp[i]);
                        dp[i] = f32_to_bf16_rne(x);
                    }
                }
            }
        }
    }
}

}  // namespace dg
