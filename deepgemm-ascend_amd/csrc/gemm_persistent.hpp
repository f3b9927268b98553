// Persistent variant of the tile kernel for the 128-K-stage tiles (two-slot late-sync ring).
//
// The grid holds at most one workgroup per CU (or per `num_cus` of set_num_sms); workgroup b
// walks the tile ids b, b + grid, b + 2 grid, ... -- each mapped to a tile exactly as a
// one-tile-per-workgroup launch maps it (XCD-aware remap, GROUP_M bands) -- so one launch
// covers every tile and the CU never idles between tiles.  The scheduler's role matches the
// reference's persistent block walk (deep_gemm/include/deep_gemm/scheduler.hpp:141-196,
// fp8_gemm.hpp:127) on CDNA4 terms.
//
// The LDS ring runs on across tiles: its loads form one stream of (tile, stage) pairs that
// stays two stages ahead of the MFMAs, so the last two stages of a tile already load the next
// tile's first two, and those loads fly while this tile's epilogue converts and stores D.
// Operand, scale and D addresses are one buffer resource per tensor with the tile's base in the
// scalar offset, so switching tiles changes a few scalars and no per-lane state.
//
// Tiles of a psum / m_indices layout that hold only padding rows are written as zeros, masked
// tiles past masked_m are skipped; both consume no stage of the load stream.
#pragma once

#include "gemm_kernel.hpp"

namespace dg {

// Scalar facts of one tile of a persistent launch.
struct PTile {
    int m0, n0, batch, group, valid_end;
    int state;   // kPCompute, kPZero (padding rows only: write zeros) or kPSkip (nothing to write)
};
constexpr int kPCompute = 0, kPZero = 1, kPSkip = 2;

template <int BM, int BN>
__device__ __forceinline__ PTile ptile_info(const KParams& p, int v, int gemm_type, int nm, int nn, int M) {
    PTile ti;
    int t = xcd_remap(v, p.num_tiles);
    ti.batch = 0;
    if (gemm_type == kBatched || gemm_type == kMasked) {
        ti.batch = t / (nm * nn);
        t -= ti.batch * nm * nn;
    }
    int mb, nb;
    swizzle_tile(t, nm, nn, p.group_m, mb, nb);
    ti.m0 = mb * BM;
    ti.n0 = nb * BN;
    ti.group = ti.batch;
    ti.valid_end = M;
    ti.state = kPCompute;
    // (the layout is read through the constant address space: scalar loads, counted apart from
    // the ring's vector-memory loads, so reading it never waits for a stage in flight)
    typedef const __attribute__((address_space(4))) int* const_ip;
    const const_ip lay = (const_ip)p.layout;
    if (gemm_type == kMasked) {
        ti.valid_end = min(M, lay[ti.batch]);
        if (ti.m0 >= ti.valid_end) ti.state = kPSkip;
    } else if (gemm_type == kMGroupedPsum) {
        // first group whose aligned end passes m0, eight psum entries per scalar round trip
        const int G = p.num_groups;
        int found = -1;
        for (int base = 0; base < G && found < 0; base += 8) {
            int e[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) e[i] = lay[min(base + i, G - 1)];
#pragma unroll
            for (int i = 0; i < 8; ++i)
                if (found < 0 && base + i < G && align_up(e[i], p.alignment) > ti.m0) found = base + i;
        }
        if (found < 0) {
            ti.state = kPZero;
        } else {
            ti.group = found;
            ti.valid_end = min(M, lay[found]);
            if (ti.valid_end <= ti.m0) ti.state = kPZero;
        }
    } else if (gemm_type == kMGroupedIdx) {
        ti.group = lay[ti.m0];
        // (padding rows, and ids past the last group -- which the m_indices check reports --
        // read no B)
        if (ti.group < 0 || ti.group >= p.num_groups) ti.state = kPZero;
    }
    ti.m0 = __builtin_amdgcn_readfirstlane(ti.m0);
    ti.n0 = __builtin_amdgcn_readfirstlane(ti.n0);
    ti.batch = __builtin_amdgcn_readfirstlane(ti.batch);
    ti.group = __builtin_amdgcn_readfirstlane(ti.group);
    ti.valid_end = __builtin_amdgcn_readfirstlane(ti.valid_end);
    ti.state = __builtin_amdgcn_readfirstlane(ti.state);
    return ti;
}

// The launch's KParams read afresh from the kernel-argument segment.  The empty asm hides the
// pointer's value from the compiler, so fields read through it at a tile boundary are loaded
// there (scalar loads) instead of being held in registers across the whole tile loop.
__device__ __forceinline__ const KParams& kparams_fresh() {
    auto kp = __builtin_amdgcn_kernarg_segment_ptr();
    asm volatile("" : "+s"(kp));
    return *(const KParams*)kp;
}

template <int BM, int BN, int WGM, int NW, int LW, int OCC, int KIND, int EPI>
__device__ __forceinline__ void gemm_persistent_body(const KParams& p) {
    constexpr int KM = 2;
    constexpr bool kAFp4 = KIND == kFP4FP4;
    constexpr bool kBFp4 = KIND == kFP8FP4 || KIND == kFP4FP4;
    constexpr bool kBf16 = KIND == kBF16;
    constexpr int kFmtA = kAFp4 ? kFmtE2M1 : kFmtE4M3;
    constexpr int kFmtB = kBFp4 ? kFmtE2M1 : kFmtE4M3;
    constexpr int KS = (kBf16 ? 32 : 64) * KM;           // K elements per stage
    constexpr int RBA = (kAFp4 ? 32 : 64) * KM;          // bytes of one row per stage
    constexpr int RBB = (kBFp4 ? 32 : 64) * KM;
    constexpr int SPRA = RBA / 16, SPRB = RBB / 16;
    constexpr int NT = NW * 64;
    constexpr int LT = LW * 64, FW = NW - LW;
    static_assert(LW == NW || (NW == 8 && LW == 4), "loader waves");
    constexpr int WGN = NW / WGM;
    constexpr int WM = BM / WGM;
    constexpr int WN = (BN / WGN + 31) / 32 * 32;
    constexpr int TM = WM / 32, TN = WN / 32;
    constexpr int TN_LAST = (BN - (WGN - 1) * WN) / 32;
    constexpr bool kRagged = TN_LAST != TN;
    static_assert((NW == 4 || NW == 8) && WGM * WGN == NW && TM >= 1 && TN >= 1 && TM * 32 == WM &&
                      TN_LAST >= 1 && (WGN - 1) * WN + TN_LAST * 32 == BN, "wave tiling");
    static_assert(!kRagged || (NW == 8 && LW == 4 && WGM == 4 && WGN == 2), "ragged tiling needs the loader waves as its last column");
    constexpr int A_BYTES = BM * RBA, B_BYTES = BN * RBB;
    constexpr int SCA = kBf16 ? 0 : (BM * 2 + 255) / 256 * 256;
    constexpr int SCB = kBf16 ? 0 : (BN * 2 + 255) / 256 * 256;
    constexpr int SCU = SCA + SCB;
    constexpr int NSCA = kBf16 ? 0 : (BM + 127) / 128, NSCB = kBf16 ? 0 : (BN + 127) / 128;
    constexpr int SPARE = (!kBf16 && NSCA + NSCB < LW) ? 256 : 0;
    constexpr int STAGE = A_BYTES + B_BYTES + KM * SCU + SPARE;
    static_assert(2 * STAGE * OCC <= 160 * 1024, "LDS budget");
    __shared__ __attribute__((aligned(1024))) uint8_t smem[2 * STAGE];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lwave = wave - FW, ltid = tid - FW * 64;
    const bool is_loader = lwave >= 0;
    const int wm = wave % WGM, wn = wave / WGM;
    const int r = lane & 31, q = lane >> 5;

    const int gemm_type = p.gemm_type;
    const int nm = p.num_m_blocks, nn = p.num_n_blocks;
    const int M = p.m, N = p.n;
    const int tiles = p.num_tiles;
    const int grid = gridDim.x;
    const int k_len = p.k;
    const int S = ceil_div(k_len, KS);                   // stages per tile
    const int nk64 = ceil_div(k_len, 64);

    // ------------------------------------------------------------------ load stream
    // One buffer resource per tensor (the host guarantees every span fits a 31-bit offset);
    // a tile's rows start at a scalar offset.  Rows past a ragged edge read the next rows of
    // the tensor (or zeros past its end): they only feed outputs that are never stored.
    const __amdgpu_buffer_rsrc_t rs_a = make_rsrc(p.a, p.a_span);
    const __amdgpu_buffer_rsrc_t rs_b = make_rsrc(p.b, p.b_span);
    const int64_t lda = p.lda, ldb = p.ldb;
    const int kbytes_a = p.kbytes_a, kbytes_b = p.kbytes_b;
    constexpr int SLA = BM * SPRA, SLB = BN * SPRB;
    constexpr int NLA = (SLA + LT - 1) / LT, NLB = (SLB + LT - 1) / LT;
    static_assert(NSCA + NSCB <= LW, "scale loads per stage");
    constexpr int NL = NLA + NLB + (kBf16 ? 0 : KM);
    constexpr int kMinLoadsPerStage = (SLA / LT) + (SLB / LT) + (kBf16 ? 0 : KM);
    int lk_a, lk_b;
    uint32_t vbase_a, vbase_b;
    {
        const int row_a = ltid / SPRA, row_b = ltid / SPRB;
        lk_a = ((ltid % SPRA) ^ slot_swizzle<SPRA>(row_a)) * 16;
        lk_b = ((ltid % SPRB) ^ slot_swizzle<SPRB>(row_b)) * 16;
        vbase_a = (uint32_t)(row_a * lda + lk_a);
        vbase_b = (uint32_t)(row_b * ldb + lk_b);
    }
    const int vstep_a = __builtin_amdgcn_readfirstlane((int)((LT / SPRA) * lda));
    const int vstep_b = __builtin_amdgcn_readfirstlane((int)((LT / SPRB) * ldb));
    __amdgpu_buffer_rsrc_t rs_sc;
    uint32_t sc_voff = kOOBOffset;
    int sc_step = 0, sc_lds = 0;
    bool sc_live = false, sc_is_a = false;
    if constexpr (!kBf16) {
        sc_is_a = lwave < NSCA;
        const int w = sc_is_a ? lwave : lwave - NSCA;
        sc_live = lwave >= 0 && lwave < NSCA + NSCB;
        rs_sc = sc_is_a ? make_rsrc(p.sfa, p.sfa_span) : make_rsrc(p.sfb, p.sfb_span);
        const int row = w * 128 + 2 * lane;
        sc_voff = sc_live && row < (sc_is_a ? BM : BN) ? (uint32_t)(row * 2) : kOOBOffset;
        sc_step = __builtin_amdgcn_readfirstlane((int)((sc_is_a ? p.sfa_ld : p.sfb_ld) * 2));
        sc_lds = __builtin_amdgcn_readfirstlane(sc_live ? A_BYTES + B_BYTES + (sc_is_a ? 0 : SCA) + w * 256
                                                        : A_BYTES + B_BYTES + KM * SCU);
    }
    constexpr int kDeadOffset = 0x40000000;

    // The stream's position: tile id ld_v (>= tiles: past the end, dead loads) and stage ld_c,
    // with that tile's scalar byte offsets into A, B and this wave's SF tensor.
    int ld_v = blockIdx.x, ld_c = 0;
    int ld_a = 0, ld_b = 0, ld_sc = 0;
    // Move to the first tile at or after ld_v that has stages to load.
    auto ld_seek = [&]() {
        for (; ld_v < tiles; ld_v += grid) {
            const KParams& pf = kparams_fresh();
            const PTile ti = ptile_info<BM, BN>(pf, ld_v, pf.gemm_type, pf.num_m_blocks, pf.num_n_blocks, pf.m);
            if (ti.state != kPCompute) continue;
            ld_a = __builtin_amdgcn_readfirstlane((int)(ti.batch * pf.bsa + (int64_t)ti.m0 * pf.lda));
            ld_b = __builtin_amdgcn_readfirstlane((int)(ti.group * pf.bsb + (int64_t)ti.n0 * pf.ldb));
            if constexpr (!kBf16)
                ld_sc = __builtin_amdgcn_readfirstlane(
                    (int)(sc_is_a ? ti.batch * pf.sfa_bs + ti.m0 : ti.group * pf.sfb_bs + ti.n0) * 2);
            return;
        }
    };
    // Issue load item IDX of the stream's next stage into ring slot s.
    auto issue_item = [&](auto idx_tag, int s) {
        const bool live = ld_v < tiles;
        uint8_t* sbase = smem + s * STAGE;
        {
            constexpr int IDX = decltype(idx_tag)::value;
            if constexpr (IDX < NLA + NLB) {
                constexpr bool kIsA = IDX < NLA;
                constexpr int it = kIsA ? IDX : IDX - NLA;
                constexpr int SL = kIsA ? SLA : SLB;
                constexpr int RB = kIsA ? RBA : RBB;
                if (SL % LT != 0 && it * LT + lwave * 64 >= SL) return;
                const int kb = ld_c * RB;
                const int krem = (kIsA ? kbytes_a : kbytes_b) - kb;
                const uint32_t voff = (kIsA ? lk_a : lk_b) < krem ? (kIsA ? vbase_a : vbase_b) : kOOBOffset;
                const int soff = (kIsA ? ld_a : ld_b) + kb + it * (kIsA ? vstep_a : vstep_b);
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    kIsA ? rs_a : rs_b, (lds_void*)(sbase + (kIsA ? 0 : A_BYTES) + (it * LT + lwave * 64) * 16), 16,
                    voff, __builtin_amdgcn_readfirstlane(live ? soff : kDeadOffset), 0, 0);
            } else if constexpr (!kBf16) {
                constexpr int u = IDX - NLA - NLB;
                const bool on = live & sc_live & (ld_c * KM + u < nk64);
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    rs_sc, (lds_void*)(sbase + sc_lds + (sc_live ? u * SCU : 0)), 4, sc_voff,
                    __builtin_amdgcn_readfirstlane(on ? ld_sc + (ld_c * KM + u) * sc_step : kDeadOffset), 0, 0);
            }
        }
    };
    // Move the stream past the stage whose items were all issued.
    auto advance = [&]() {
        if (ld_v < tiles && ++ld_c == S) {
            ld_c = 0;
            ld_v += grid;
            ld_seek();
        }
    };
    auto issue_next = [&](int s) {
        static_for<NL>([&](auto i) { issue_item(i, s); });
        advance();
    };

    // ------------------------------------------------------------------ fragments
    auto frag_addr = [&](int R, int slot, auto spr_tag) -> int {
        constexpr int SPR = decltype(spr_tag)::value;
        return R * (SPR * 16) + ((slot ^ slot_swizzle<SPR>(R)) << 4);
    };
    auto load_frag = [&](const uint8_t* base, int R, auto spr_tag, auto u_tag) -> i32x8 {
        constexpr int SPR = decltype(spr_tag)::value;
        constexpr int u = decltype(u_tag)::value;
        constexpr int P = SPR / KM;
        const i32x4 lo = *reinterpret_cast<const i32x4*>(base + frag_addr(R, u * P + q, spr_tag));
        if constexpr (P == 4) {
            const i32x4 hi = *reinterpret_cast<const i32x4*>(base + frag_addr(R, u * P + 2 + q, spr_tag));
            return i32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        } else {
            return i32x8{lo[0], lo[1], lo[2], lo[3], 0, 0, 0, 0};
        }
    };
    auto load_scale = [&](const uint8_t* sc, int R) -> int { return sc[R * 2 + q]; };

    f32x16 acc[TN][TM];
    i32x8 fa[2][TM];
    int sa[2][TM];
    i32x8 fb0[2];
    int sb0[2];
    auto prefetch = [&](int s, auto buf_tag, auto part_tag, auto u_tag) {
        constexpr int buf = decltype(buf_tag)::value;
        constexpr int part = decltype(part_tag)::value;
        constexpr int u = decltype(u_tag)::value;
        const uint8_t* st = smem + s * STAGE;
        const uint8_t* sc = st + A_BYTES + B_BYTES + u * SCU;
        if constexpr (part < TM) {
            const int R = wm * WM + part * 32 + r;
            fa[buf][part] = load_frag(st, R, Int<SPRA>{}, u_tag);
            sa[buf][part] = kBf16 ? 0 : load_scale(sc, R);
        } else {
            const int R = wn * WN + r;
            fb0[buf] = load_frag(st + A_BYTES, R, Int<SPRB>{}, u_tag);
            sb0[buf] = kBf16 ? 0 : load_scale(sc + SCA, R);
        }
    };

    // Sub-step u of the stage in slot s (register set u).  Sub-step 0 reads sub-step 1's ahead
    // registers; sub-step 1 syncs late: once its last fragments are in registers, before its
    // last MFMA group, the waves wait for the next stage (slot s ^ 1), meet at the barrier, read
    // its first fragments and refill slot s with the stream's next stage.
    // kLast (the tile's last stage) leaves the next stage's first fragments unread: the epilogue
    // runs with them out of registers and the next tile reads them afterwards.
    auto compute = [&](int s, auto u_tag, auto loads_tag, auto tnx_tag, auto last_tag) {
        constexpr int u = decltype(u_tag)::value;
        constexpr bool kLast = decltype(last_tag)::value != 0;
        constexpr bool kLoadWave = decltype(loads_tag)::value != 0;
        constexpr int TNX = decltype(tnx_tag)::value;
        const uint8_t* sB = smem + s * STAGE + A_BYTES;
        const uint8_t* sSB = smem + s * STAGE + A_BYTES + B_BYTES + u * SCU + SCA;
        i32x8 fb_cur = fb0[u];
        int sb_cur = sb0[u];
        static_for<TNX>([&](auto jn_c) {
            constexpr int jn = decltype(jn_c)::value;
            i32x8 fb_next = fb_cur;
            int sb_next = sb_cur;
            if constexpr (jn + 1 < TNX) {
                fb_next = load_frag(sB, wn * WN + (jn + 1) * 32 + r, Int<SPRB>{}, u_tag);
                if constexpr (!kBf16) sb_next = load_scale(sSB, wn * WN + (jn + 1) * 32 + r);
            }
            if constexpr (u == 1 && jn + 1 == TNX) {
                wait_vmcnt<0>();
                stage_barrier();
                if constexpr (!kLast)
                    static_for<TM + 1>([&](auto part_c) { prefetch(s ^ 1, Int<0>{}, part_c, Int<0>{}); });
                __builtin_amdgcn_sched_barrier(0);
                if constexpr (kLoadWave) issue_next(s);
            }
            static_for<TM>([&](auto jm_c) {
                constexpr int jm = decltype(jm_c)::value;
                if constexpr (kBf16) {
                    const i32x4 b0 = {fb_cur[0], fb_cur[1], fb_cur[2], fb_cur[3]};
                    const i32x4 b1 = {fb_cur[4], fb_cur[5], fb_cur[6], fb_cur[7]};
                    const i32x4 a0 = {fa[u][jm][0], fa[u][jm][1], fa[u][jm][2], fa[u][jm][3]};
                    const i32x4 a1 = {fa[u][jm][4], fa[u][jm][5], fa[u][jm][6], fa[u][jm][7]};
                    acc[jn][jm] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                        __builtin_bit_cast(bf16x8, b0), __builtin_bit_cast(bf16x8, a0), acc[jn][jm], 0, 0, 0);
                    acc[jn][jm] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                        __builtin_bit_cast(bf16x8, b1), __builtin_bit_cast(bf16x8, a1), acc[jn][jm], 0, 0, 0);
                } else {
                    acc[jn][jm] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
                        fb_cur, fa[u][jm], acc[jn][jm], kFmtB, kFmtA, 0, sb_cur, 0, sa[u][jm]);
                }
            });
            if constexpr (u == 0) {
                // sub-step 1's ahead registers: A block jm goes with group jm * TNX / TM, the first
                // B block with the last group
                static_for<TM + 1>([&](auto part_c) {
                    constexpr int part = decltype(part_c)::value;
                    constexpr int grp = part < TM ? part * TNX / TM : TNX - 1;
                    if constexpr (grp == jn) prefetch(s, Int<1>{}, Int<part>{}, Int<1>{});
                });
            }
            __builtin_amdgcn_sched_barrier(0);
            fb_cur = fb_next;
            sb_cur = sb_next;
        });
    };

    // ------------------------------------------------------------------ tile loop
    // Prologue: the stream's first two stages in flight, the first one visible and its first
    // fragments in registers.
    ld_seek();
    if (is_loader) {
        issue_next(0);
        issue_next(1);
    }
    wait_vmcnt<kMinLoadsPerStage>();
    stage_barrier();

    auto tile_loop = [&](auto loads_tag, auto tnx_tag) {
        int s = 0;   // ring slot of the next stage to compute
        for (int v = blockIdx.x; v < tiles; v += grid) {
            const KParams& pf = kparams_fresh();
            const PTile ti = ptile_info<BM, BN>(pf, v, pf.gemm_type, pf.num_m_blocks, pf.num_n_blocks, pf.m);
            uint8_t* d_base = pf.d + (int64_t)ti.batch * pf.bsd * pf.out_esize;
            if (ti.state == kPSkip) continue;
            if (ti.state == kPZero) {
                const int rows = min(BM, pf.m - ti.m0), cols = min(BN, pf.n - ti.n0);
                for (int e = tid; e < rows * cols; e += NT) {
                    const int rr = e / cols, cc = e % cols;
                    const int64_t off = (int64_t)(ti.m0 + rr) * pf.ldd + ti.n0 + cc;
                    if (pf.out_esize == 4) reinterpret_cast<float*>(d_base)[off] = 0.f;
                    else reinterpret_cast<uint16_t*>(d_base)[off] = 0;
                }
                continue;
            }
#pragma unroll
            for (int i = 0; i < TN; ++i)
#pragma unroll
                for (int j = 0; j < TM; ++j) acc[i][j] = f32x16{};
            // the tile's first fragments (its first stage is visible: the prologue or the previous
            // tile's last barrier waited for it)
            static_for<TM + 1>([&](auto part_c) { prefetch(s, Int<0>{}, part_c, Int<0>{}); });
            for (int c = 0; c + 1 < S; ++c) {
                compute(s, Int<0>{}, loads_tag, tnx_tag, Int<0>{});
                compute(s, Int<1>{}, loads_tag, tnx_tag, Int<0>{});
                s ^= 1;
            }
            compute(s, Int<0>{}, loads_tag, tnx_tag, Int<1>{});
            compute(s, Int<1>{}, loads_tag, tnx_tag, Int<1>{});
            s ^= 1;
            const KParams& pe = kparams_fresh();
            // (lane coordinates laundered here, so the compiler derives the epilogue's per-lane
            // addresses at each tile's end instead of keeping them live across the main loop)
            int er = r, eq = q;
            asm volatile("" : "+v"(er), "+v"(eq));
            static_for<TM>([&](auto jm_c) {
                constexpr int jm = decltype(jm_c)::value;
                const int m = ti.m0 + wm * WM + jm * 32 + er;
                const bool row_ok = m < pe.m && !(pe.gemm_type == kMasked && m >= ti.valid_end);
                bool pad_row = false;
                if (pe.gemm_type == kMGroupedPsum) pad_row = m >= ti.valid_end;
                else if (pe.gemm_type == kMGroupedIdx) pad_row = row_ok && pe.layout[m] != ti.group;
                static_for<TN>([&](auto jn_c) {
                    constexpr int jn = decltype(jn_c)::value;
                    if (kRagged && jn >= TN_LAST && wn == WGN - 1) return;
                    epilogue_block<EPI>(pe, acc[jn][jm], d_base, m, row_ok, pad_row, ti.n0 + wn * WN + jn * 32, pe.n,
                                        ti.batch, eq);
                });
            });
        }
    };
    if (LW == NW || is_loader) tile_loop(Int<1>{}, Int<TN_LAST>{});
    else tile_loop(Int<0>{}, Int<TN>{});
    __builtin_amdgcn_s_waitcnt(0);
}

template <int BM, int BN, int WGM, int NW, int LW, int OCC, int KIND, int EPI>
__global__ __launch_bounds__(NW * 64, OCC * NW / 4) void gemm_persistent_kernel(const KParams p) {
    gemm_persistent_body<BM, BN, WGM, NW, LW, OCC, KIND, EPI>(p);
}

}  // namespace dg
