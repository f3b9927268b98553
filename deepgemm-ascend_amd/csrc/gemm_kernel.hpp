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

#include <type_traits>
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
    unsigned long long* dbg_ts;  // profiling: per-workgroup timestamps (null = off)
    int dbg;                   // profiling switch: 1 = skip operand loads, 2 = skip MFMA,
                               // 3 = skip scale loads, 4 = skip all loads, 5 = epilogue only
};

// Epilogue variants.
constexpr int kEpiLdsBf16 = 0;   // bf16 D, no accumulation, 16-byte aligned rows
constexpr int kEpiF32 = 1;       // fp32 D (bias / accumulate allowed)
constexpr int kEpiBf16 = 2;      // bf16 D with accumulation or unaligned rows

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
// Chosen so that the 16 rows one ds_read_b128 phase touches (lanes r = 0..15 at a fixed lane
// group) land on distinct 16-byte bank groups both for a 64 x 4-byte and a 32 x 4-byte bank
// organisation.
template <int SPR>
__device__ __forceinline__ int slot_swizzle(int row) {
    if constexpr (SPR == 8) return ((row >> 1) ^ (row << 2)) & 7;
    else return ((row >> 1) ^ (row >> 3)) & 3;
}

// Buffer resource over [base, base + bytes); every field is forced wave-uniform (SGPRs) so no
// buffer instruction using it ever needs a waterfall loop.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, int64_t bytes) {
    if (bytes > 0x7fffffffLL) bytes = 0x7fffffffLL;
    if (bytes < 0) bytes = 0;
    const uint64_t addr = reinterpret_cast<uint64_t>(base);
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)addr);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(addr >> 32));
    const int nbytes = __builtin_amdgcn_readfirstlane((int)bytes);
    void* ub = reinterpret_cast<void*>(((uint64_t)hi << 32) | lo);
    return __builtin_amdgcn_make_buffer_rsrc(ub, (short)0, nbytes, (int)kBufferRsrcWord3);
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

template <int BM, int BN, int KIND, int EPI>
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
    constexpr int CROW = BN * 2 + 32;                       // LDS row pitch of the bf16 epilogue tile
    constexpr int EPI_BYTES = EPI == kEpiLdsBf16 ? BM * CROW : 0;
    constexpr int SMEM = 2 * STAGE > EPI_BYTES ? 2 * STAGE : EPI_BYTES;
    __shared__ __attribute__((aligned(1024))) uint8_t smem[SMEM];

    const int tid = threadIdx.x;
    unsigned long long* ts = p.dbg_ts ? p.dbg_ts + (size_t)blockIdx.x * 8 : nullptr;
    auto stamp = [&](int i) { if (ts && tid == 0) ts[i] = __builtin_amdgcn_s_memrealtime(); };
    stamp(0);
    if (ts && tid == 0) ts[2] = __builtin_amdgcn_s_getreg((4 << 0) | (0 << 6) | (31 << 11));  // HW_ID
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
        group = __builtin_amdgcn_readfirstlane(p.layout[m0]);
        if (group < 0) zero_tile = true;
    }

    group = __builtin_amdgcn_readfirstlane(group);
    valid_end = __builtin_amdgcn_readfirstlane(valid_end);
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
    const int num_chunks = p.dbg == 11 ? 0 : ceil_div(p.k, KC);
    const int nk64 = ceil_div(p.k, 64);

    // ------------------------------------------------------------------ loaders
    // Operand tiles: each wave-level buffer_load_dwordx4 ... lds fills 1 KB (64 lanes x 16 B)
    // of an LDS stage; lane slots map to XOR-swizzled (row, 16-byte K piece) positions.  The
    // chunk's K offset rides in the scalar soffset so the per-lane voffset is chunk-invariant,
    // and the lane index is made opaque to the optimiser so that voffset is recomputed (a few
    // VALU ops) instead of being hoisted into long-lived VGPRs.
    constexpr int NLA = A_BYTES / 4096 + (A_BYTES % 4096 ? 1 : 0);   // loads per wave, A tile
    constexpr int NLB = B_BYTES / 4096 + (B_BYTES % 4096 ? 1 : 0);   // loads per wave, B tile
    constexpr int NL = NLA + NLB;
    // Per-load chunk-invariant voffsets (row * ld + swizzled K piece, or out of range).
    auto load_geom = [&](auto idx_tag, int t, int& row, int& lk) {
        constexpr int IDX = decltype(idx_tag)::value;
        constexpr bool kIsA = IDX < NLA;
        constexpr int it = kIsA ? IDX : IDX - NLA;
        constexpr int SPR = kIsA ? SPRA : SPRB;
        const int slot = it * 256 + t;
        row = slot / SPR;
        lk = ((slot % SPR) ^ slot_swizzle<SPR>(row)) * 16;
    };
    uint32_t voff_pre[NL];
    static_for<NL>([&](auto i) {
        constexpr int IDX = decltype(i)::value;
        constexpr bool kIsA = IDX < NLA;
        int row, lk;
        load_geom(i, tid, row, lk);
        voff_pre[IDX] = row < (kIsA ? rows_a : rows_b) ? (uint32_t)(row * (kIsA ? lda : ldb) + lk) : kOOBOffset;
    });
    // The swizzled K piece of a lane's slot is the same for every load of one operand (the
    // swizzle only reads row bits that a whole 4 KB load block leaves unchanged).
    int lk_a, lk_b, row_unused;
    load_geom(Int<0>{}, tid, row_unused, lk_a);
    load_geom(Int<NLA>{}, tid, row_unused, lk_b);
    // Loads of chunk c into stage s.  Branch-free so the scheduler can interleave them with
    // MFMAs: `live == false` moves every lane out of range through the scalar offset (no
    // memory traffic, zeros into an idle stage); K-tail pieces go out of range per lane.
    constexpr int kDeadOffset = 0x40000000;
    auto issue_one = [&](auto idx_tag, int c, int s, bool live) {
        constexpr int IDX = decltype(idx_tag)::value;
        constexpr bool kIsA = IDX < NLA;
        constexpr int it = kIsA ? IDX : IDX - NLA;
        constexpr int BYTES = kIsA ? A_BYTES : B_BYTES;
        constexpr int RB = kIsA ? RBA : RBB;
        if (BYTES % 4096 != 0 && (it * 256 + wave * 64) * 16 >= BYTES) return;
        const int kb = (p.dbg == 9 ? 0 : c) * RB;
        const int krem = (kIsA ? kbytes_a : kbytes_b) - kb;
        const uint32_t voff = (kIsA ? lk_a : lk_b) < krem ? voff_pre[IDX] : kOOBOffset;
        uint8_t* sdst = smem + s * STAGE + (kIsA ? 0 : A_BYTES);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(kIsA ? rs_a : rs_b,
                                                 (lds_void*)(sdst + (it * 256 + wave * 64) * 16), 16, voff,
                                                 live ? kb : kDeadOffset, 0, 0);
    };
    auto issue_data = [&](int c, int s) {
        static_for<NL>([&](auto i) { issue_one(i, c, s, true); });
    };

    // Scales: the two packed int16 rows (k64 = 2c, 2c+1) of this chunk for the tile's rows,
    // through buffer loads (out-of-range rows / K blocks read 0: their operand data is 0 too).
    constexpr int NSA = (2 * BM + 255) / 256, NSB = (2 * BN + 255) / 256;
    uint32_t sa_reg[NSA], sb_reg[NSB];
    __amdgpu_buffer_rsrc_t rs_sa, rs_sb;
    if constexpr (!kBf16) {
        rs_sa = make_rsrc(sfa + m0, ((int64_t)nk64 * p.sfa_ld - m0) * 2);
        rs_sb = make_rsrc(sfb + n0, ((int64_t)nk64 * p.sfb_ld - n0) * 2);
    }
    // byte distance between the packed-SF rows of consecutive chunks (two int16 rows)
    const int sfa_step = __builtin_amdgcn_readfirstlane((int)(p.sfa_ld * 4));
    const int sfb_step = __builtin_amdgcn_readfirstlane((int)(p.sfb_ld * 4));
    auto issue_scales = [&](int c, bool live) {
        if constexpr (!kBf16) {
#pragma unroll
            for (int i = 0; i < NSA; ++i) {
                const int idx = i * 256 + tid;
                const int h = idx / BM, row = idx % BM;
                const uint32_t voff = idx < 2 * BM ? (uint32_t)((h * p.sfa_ld + row) * 2) : kOOBOffset;
                sa_reg[i] = __builtin_amdgcn_raw_buffer_load_b16(rs_sa, voff, live ? c * sfa_step : kDeadOffset, 0);
            }
#pragma unroll
            for (int i = 0; i < NSB; ++i) {
                const int idx = i * 256 + tid;
                const int h = idx / BN, row = idx % BN;
                const uint32_t voff = idx < 2 * BN ? (uint32_t)((h * p.sfb_ld + row) * 2) : kOOBOffset;
                sb_reg[i] = __builtin_amdgcn_raw_buffer_load_b16(rs_sb, voff, live ? c * sfb_step : kDeadOffset, 0);
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

    // One K chunk of MFMAs from LDS stage s.  When `next` is set, the loads of chunk c + 1
    // (into stage s ^ 1) are interleaved with the MFMA groups: a buffer_load ... lds blocks
    // issue while the texture path drains, so issuing them in one burst would stall the MFMA
    // pipe.  They go out over the first groups to leave latency slack before the next wait.
    constexpr int kLoadGroups = TN > 2 ? (TN * 2 + 2) / 3 : TN;
    constexpr int kLPG = (NL + kLoadGroups - 1) / kLoadGroups;    // loads per MFMA group
    auto compute = [&](int s, int cn, bool next) {
        const uint8_t* sA = smem + s * STAGE;
        const uint8_t* sB = sA + A_BYTES;
        i32x8 fa[TM];
#pragma unroll
        for (int jm = 0; jm < TM; ++jm) fa[jm] = load_frag(sA, wm * WM + jm * 16 + r, Int<SPRA>{});
        i32x2 sa2 = {0, 0}, sb2 = {0, 0};
        if constexpr (!kBf16) {
            const uint8_t* sSA = sA + A_BYTES + B_BYTES;
            const uint8_t* sSB = sSA + SC_BYTES;
            sa2 = *reinterpret_cast<const i32x2*>(sSA + (q * 16 + r) * 16 + wm * 8);
            sb2 = *reinterpret_cast<const i32x2*>(sSB + (q * 16 + r) * 16 + wn * 8);
        }
        i32x8 fb_cur = load_frag(sB, wn * WN + r, Int<SPRB>{});
        static_for<TN>([&](auto jn_c) {
            constexpr int jn = decltype(jn_c)::value;
            i32x8 fb_next = fb_cur;
            if constexpr (jn + 1 < TN) fb_next = load_frag(sB, wn * WN + (jn + 1) * 16 + r, Int<SPRB>{});
            static_for<TM>([&](auto jm_c) {
                constexpr int jm = decltype(jm_c)::value;
                if constexpr (kBf16) {
                    const i32x4 blo = {fb_cur[0], fb_cur[1], fb_cur[2], fb_cur[3]};
                    const i32x4 bhi = {fb_cur[4], fb_cur[5], fb_cur[6], fb_cur[7]};
                    const i32x4 alo = {fa[jm][0], fa[jm][1], fa[jm][2], fa[jm][3]};
                    const i32x4 ahi = {fa[jm][4], fa[jm][5], fa[jm][6], fa[jm][7]};
                    acc[jn][jm] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                        __builtin_bit_cast(bf16x8, blo), __builtin_bit_cast(bf16x8, alo), acc[jn][jm], 0, 0, 0);
                    acc[jn][jm] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                        __builtin_bit_cast(bf16x8, bhi), __builtin_bit_cast(bf16x8, ahi), acc[jn][jm], 0, 0, 0);
                } else {
                    acc[jn][jm] = mfma_scaled<kFmtB, kFmtA, jn % 4, jm % 4>(
                        fb_cur, fa[jm], acc[jn][jm], sb2[jn / 4], sa2[jm / 4]);
                }
            });
            constexpr int kScaleLoads = (!kBf16 && jn == 0) ? NSA + NSB : 0;
            constexpr int kVmem = (jn * kLPG >= NL ? 0 : (NL - jn * kLPG < kLPG ? NL - jn * kLPG : kLPG)) + kScaleLoads;
            constexpr int kDs = jn + 1 < TN ? 2 : 0;
            if constexpr (jn == 0) issue_scales(cn, next);
            static_for<kLPG>([&](auto li) {
                constexpr int idx = jn * kLPG + decltype(li)::value;
                if constexpr (idx < NL) issue_one(Int<idx>{}, cn, s ^ 1, next);
            });
            // interleave: each MFMA is followed by at most one LDS read and one buffer load
            static_for<TM>([&](auto i_c) {
                constexpr int i = decltype(i_c)::value;
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                if constexpr (i < kDs) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                if constexpr (i < kVmem) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
            });
            __builtin_amdgcn_sched_barrier(0);
            fb_cur = fb_next;
        });
    };

    // ------------------------------------------------------------------ main loop
    if (num_chunks > 0) {
        issue_data(0, 0);
        issue_scales(0, true);
    }
    for (int c = 0; c < num_chunks; ++c) {
        const int s = c & 1;
        __builtin_amdgcn_s_waitcnt(0);   // chunk c data (LDS) and scales (VGPR) have landed
        write_scales(s);
        __syncthreads();
        compute(s, c + 1, c + 1 < num_chunks && p.dbg != 10);
    }
    // ------------------------------------------------------------------ epilogue
    // All accumulator indexing below is in compile-time-unrolled loops (static_for): a
    // runtime index would demote the accumulator array to scratch memory.
    const float alpha = p.alpha;
    if constexpr (EPI == kEpiLdsBf16) {
        // bf16 D without accumulation: alpha / bias / padding-row zeroing in registers, the
        // tile staged through LDS as bf16, then written with 16-byte row-contiguous stores.
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();                                     // all waves are done with the operands
        const bool bias = p.has_bias;
        const uint16_t* bp = reinterpret_cast<const uint16_t*>(p.bias);
        static_for<TM>([&](auto jm_c) {
            constexpr int jm = decltype(jm_c)::value;
            const int ml = wm * WM + jm * 16 + r;
            const int m = m0 + ml;
            bool zero = false;
            if (p.gemm_type == kMGroupedPsum) zero = m >= valid_end;
            else if (p.gemm_type == kMGroupedIdx) zero = m < M && p.layout[m] != group;
            static_for<TN>([&](auto jn_c) {
                constexpr int jn = decltype(jn_c)::value;
                const int nl = wn * WN + jn * 16 + 4 * q;
                float v0 = acc[jn][jm][0] * alpha, v1 = acc[jn][jm][1] * alpha;
                float v2 = acc[jn][jm][2] * alpha, v3 = acc[jn][jm][3] * alpha;
                if (bias) {
                    const int n = n0 + nl;
                    v0 += n + 0 < N ? bf16_to_f32(bp[n + 0]) : 0.f;
                    v1 += n + 1 < N ? bf16_to_f32(bp[n + 1]) : 0.f;
                    v2 += n + 2 < N ? bf16_to_f32(bp[n + 2]) : 0.f;
                    v3 += n + 3 < N ? bf16_to_f32(bp[n + 3]) : 0.f;
                }
                uint32_t lo = pack_bf16x2(v0, v1);
                uint32_t hi = pack_bf16x2(v2, v3);
                if (zero) lo = hi = 0;
                *reinterpret_cast<i32x2*>(smem + ml * CROW + nl * 2) = i32x2{(int)lo, (int)hi};
            });
        });
        __syncthreads();
        const int rows = min(BM, (p.gemm_type == kMasked ? valid_end : M) - m0);
        const int cols = min(BN, N - n0);
        constexpr int CPR = BN * 2 / 16;                     // 16-byte chunks per tile row
        uint16_t* dbase = reinterpret_cast<uint16_t*>(d_base);
        for (int e = tid; e < BM * CPR; e += 256) {
            const int row = e / CPR, ch = e % CPR;
            if (row >= rows) break;
            const int col = ch * 8;
            if (col >= cols) continue;
            const i32x4 val = *reinterpret_cast<const i32x4*>(smem + row * CROW + ch * 16);
            uint16_t* dp = dbase + (int64_t)(m0 + row) * p.ldd + n0 + col;
            if (col + 8 <= cols) {
                *reinterpret_cast<i32x4*>(dp) = val;
            } else {
                const uint16_t* hv = reinterpret_cast<const uint16_t*>(&val);
                for (int i = 0; i < cols - col; ++i) dp[i] = hv[i];
            }
        }
        stamp(1);
    } else {
        // fp32 D (EPI == kEpiF32) or bf16 D with accumulation / unaligned rows (kEpiBf16):
        // direct stores of each lane's four consecutive columns.
        constexpr bool kF32 = EPI == kEpiF32;
        using OutT = std::conditional_t<kF32, float, uint16_t>;
        OutT* dbase = reinterpret_cast<OutT*>(d_base);
        const OutT* bp = reinterpret_cast<const OutT*>(p.bias);
        const bool acc_old = p.accumulate, bias = p.has_bias, vec = p.vec_store;
        static_for<TM>([&](auto jm_c) {
            constexpr int jm = decltype(jm_c)::value;
            const int m = m0 + wm * WM + jm * 16 + r;
            const bool row_ok = m < M && !(p.gemm_type == kMasked && m >= valid_end);
            bool pad_row = false;
            if (p.gemm_type == kMGroupedPsum) pad_row = m >= valid_end;
            else if (p.gemm_type == kMGroupedIdx) pad_row = row_ok && p.layout[m] != group;
            OutT* drow = dbase + (int64_t)m * p.ldd;
            if constexpr (kF32) {
                static_for<TN>([&](auto jn_c) {
                    constexpr int jn = decltype(jn_c)::value;
                    const int nb = n0 + wn * WN + jn * 16 + 4 * q;
                    float v[4] = {acc[jn][jm][0] * alpha, acc[jn][jm][1] * alpha,
                                  acc[jn][jm][2] * alpha, acc[jn][jm][3] * alpha};
                    if (row_ok && nb < N) {
                        float* dp = drow + nb;
                        if (vec && nb + 3 < N) {
                            f32x4 o = {v[0], v[1], v[2], v[3]};
                            if (bias) o += f32x4{bp[nb], bp[nb + 1], bp[nb + 2], bp[nb + 3]};
                            if (acc_old) o += *reinterpret_cast<const f32x4*>(dp);
                            if (pad_row) o = f32x4{0.f, 0.f, 0.f, 0.f};
                            *reinterpret_cast<f32x4*>(dp) = o;
                        } else {
                            for (int i = 0; i < 4 && nb + i < N; ++i) {
                                float x = v[i];
                                if (bias) x += bp[nb + i];
                                if (acc_old) x += dp[i];
                                dp[i] = pad_row ? 0.f : x;
                            }
                        }
                    }
                });
            } else {
                // Round every block to bf16 pairs (bias / accumulation in fp32 first).
                uint32_t pk[TN][2];
                static_for<TN>([&](auto jn_c) {
                    constexpr int jn = decltype(jn_c)::value;
                    const int nb = n0 + wn * WN + jn * 16 + 4 * q;
                    float v[4] = {acc[jn][jm][0] * alpha, acc[jn][jm][1] * alpha,
                                  acc[jn][jm][2] * alpha, acc[jn][jm][3] * alpha};
                    const bool full = vec && nb + 3 < N;
                    if (bias) {
                        if (full) {
                            const i32x2 b2 = *reinterpret_cast<const i32x2*>(bp + nb);
                            v[0] += bf16_to_f32((uint16_t)(b2[0] & 0xffff));
                            v[1] += bf16_to_f32((uint16_t)((uint32_t)b2[0] >> 16));
                            v[2] += bf16_to_f32((uint16_t)(b2[1] & 0xffff));
                            v[3] += bf16_to_f32((uint16_t)((uint32_t)b2[1] >> 16));
                        } else {
                            for (int i = 0; i < 4; ++i) v[i] += nb + i < N ? bf16_to_f32(bp[nb + i]) : 0.f;
                        }
                    }
                    if (acc_old && row_ok) {
                        if (full) {
                            const i32x2 o2 = *reinterpret_cast<const i32x2*>(drow + nb);
                            v[0] += bf16_to_f32((uint16_t)(o2[0] & 0xffff));
                            v[1] += bf16_to_f32((uint16_t)((uint32_t)o2[0] >> 16));
                            v[2] += bf16_to_f32((uint16_t)(o2[1] & 0xffff));
                            v[3] += bf16_to_f32((uint16_t)((uint32_t)o2[1] >> 16));
                        } else {
                            for (int i = 0; i < 4; ++i) v[i] += nb + i < N ? bf16_to_f32(drow[nb + i]) : 0.f;
                        }
                    }
                    pk[jn][0] = pad_row ? 0u : pack_bf16x2(v[0], v[1]);
                    pk[jn][1] = pad_row ? 0u : pack_bf16x2(v[2], v[3]);
                });
                // Stores.  Two n-blocks (jn0, jn0 + 1) are regrouped across the lane halves of
                // each 32-lane row with v_permlane16_swap so that every lane owns 8 consecutive
                // columns: one 16-byte store per lane, 64 contiguous bytes per row.
                auto store8 = [&](auto jn_c) {
                    constexpr int jn = decltype(jn_c)::value;
                    const int nb = n0 + wn * WN + jn * 16 + 4 * q;
                    if (!row_ok || nb >= N) return;
                    uint16_t* dp = drow + nb;
                    if (vec && nb + 3 < N) {
                        *reinterpret_cast<i32x2*>(dp) = i32x2{(int)pk[jn][0], (int)pk[jn][1]};
                    } else {
                        for (int i = 0; i < 4 && nb + i < N; ++i)
                            dp[i] = (uint16_t)(pk[jn][i >> 1] >> ((i & 1) * 16));
                    }
                };
                static_for<(TN + 1) / 2>([&](auto jp_c) {
                    constexpr int jn0 = 2 * decltype(jp_c)::value;
                    if constexpr (jn0 + 1 < TN) {
                        const int nbase = n0 + wn * WN + jn0 * 16;      // wave-uniform
                        if (vec && nbase + 32 <= N) {
                            const auto s0 = __builtin_amdgcn_permlane16_swap(pk[jn0][0], pk[jn0 + 1][0], false, false);
                            const auto s1 = __builtin_amdgcn_permlane16_swap(pk[jn0][1], pk[jn0 + 1][1], false, false);
                            const int ncol = nbase + ((q & 1) ? 16 + 4 * (q - 1) : 4 * q);
                            if (row_ok)
                                *reinterpret_cast<i32x4*>(drow + ncol) =
                                    i32x4{(int)s0[0], (int)s1[0], (int)s0[1], (int)s1[1]};
                        } else {
                            store8(Int<jn0>{});
                            store8(Int<jn0 + 1>{});
                        }
                    } else {
                        store8(Int<jn0>{});
                    }
                });
            }
        });
    }
}

}  // namespace dg
