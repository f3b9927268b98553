// Skinny-M GEMM kernel for gfx950 (decode shapes: the whole of M fits one 32 MT-row tile).
//
// Same contract as gemm_kernel (D = alpha * A . B^T (+ bias | + D), per-32-K UE8M0 scales, the
// epilogue variants of epilogue_block) for dense, batched and M-grouped masked GEMMs,
// specialised for M <= 32 MT (masked: max_m), where the GEMM is a stream of B through the CUs
// and the tile kernel's LDS ring cannot keep enough bytes in flight.
//
// A workgroup owns one 32 NB-column strip of D (all M rows).  Its NW waves split the strip's K
// range between them in contiguous runs of groups of G 64-K blocks.  Each wave has a private
// ring of D group slots in LDS that it fills with whole-line global->LDS loads (buffer_load ...
// lds: one instruction moves 8 rows x 128 bytes) and reads back in the MFMA operand layout
// (ds_read_b128, the tile kernel's bank swizzle); no other wave touches the ring, so the main
// loop has no workgroup barrier, only vmcnt waits.  The first AR rows of A travel the same way (rows of
// the 32 MT-row tile past AR are zeros: AR is sized to the M the configuration serves), the
// scales go straight to registers.  While group i runs its MFMAs, groups i + 1 .. i + D - 1
// are in flight.  At the end the waves' partial tiles meet in LDS and are summed in wave
// order (deterministic).  Long K with few strips is also cut across workgroups (split-K
// through a workspace, as in gemm_kernel: the last workgroup of a strip sums the partials in
// split order).
//
// MFMA operand layout (see gemm_kernel.hpp): for each 64-K block lane (r, q) needs, of row r,
// the 16-byte pieces at bytes 32 j + 16 q (j < 2 for e4m3, j < 1 for e2m1; bf16: j < 4, one
// per 32x32x16 K-step) and the UE8M0 byte q of the row's packed scale pair (int16 per row and
// 64-K block, the low byte for K [0, 32)).
#pragma once

#include "gemm_kernel.hpp"

namespace dg {

// Ring geometry of a skinny kernel configuration (host and device).
struct SkinnyShape {
    int g;       // 64-K blocks per group (a group row is 128 bytes for e4m3 / bf16, 64 for e2m1)
    int rg;      // bytes of one B row in a group slot
    int rga;     // bytes of one A row in a group slot
    int loads;   // vector-memory instructions per group: B and A rows (1 KB each), scale dwords
};
__host__ __device__ constexpr SkinnyShape skinny_shape(int kind, int mt, int nb, int ar) {
    const int g = kind == kBF16 ? 1 : 2;
    const int rg = g * (kind == kBF16 ? 128 : (kind == kFP8FP8 ? 64 : 32));
    const int rga = g * (kind == kBF16 ? 128 : (kind == kFP4FP4 ? 32 : 64));
    return {g, rg, rga, (nb * 32 * rg + ar * rga) / 1024 + (kind == kBF16 ? 0 : g * (nb + mt))};
}

// x >> sh, kept at its place in the instruction stream (volatile), so the compiler cannot move
// it to where the loaded x has not been waited for yet.
__device__ __forceinline__ int shift_at_use(int x, int sh) {
    int y;
    asm volatile("v_lshrrev_b32 %0, %1, %2" : "=v"(y) : "v"(sh), "v"(x));
    return y;
}

template <int KIND, int MT, int NB, int NW, int D, int AR, int EPI, bool BMN = false>
__device__ __forceinline__ void skinny_body(const KParams& p, const int vb) {
    constexpr bool kAFp4 = KIND == kFP4FP4;
    constexpr bool kBFp4 = KIND == kFP8FP4 || KIND == kFP4FP4;
    constexpr bool kBf16 = KIND == kBF16;
    constexpr int kFmtA = kAFp4 ? kFmtE2M1 : kFmtE4M3;
    constexpr int kFmtB = kBFp4 ? kFmtE2M1 : kFmtE4M3;
    constexpr int BM = 32 * MT, BN = 32 * NB;
    constexpr int RBA = kBf16 ? 128 : (kAFp4 ? 32 : 64);   // bytes of one row per 64-K block
    constexpr int RBB = kBf16 ? 128 : (kBFp4 ? 32 : 64);
    constexpr int PA = RBA / 32, PB = RBB / 32;            // 16-byte pieces per lane and block
    constexpr SkinnyShape kShape = skinny_shape(KIND, MT, NB, AR);
    constexpr int G = kShape.g, RG = kShape.rg, RGA = kShape.rga;
    constexpr int SPR = RG / 16, SPRA = RGA / 16;           // 16-byte slots of a B / A row
    constexpr int RPI = 64 / SPR, RPIA = 64 / SPRA;         // rows per load instruction
    constexpr int NDMA = BN / RPI, NDMAA = AR / RPIA;       // load instructions per group slot
    static_assert(AR % RPIA == 0 && AR <= BM, "staged A rows");
    // MN-major B (BMN: B stored [K][N], N contiguous; e4m3 or bf16, one 32-column block per strip): a
    // group slot holds the group's K rows of the strip's 32 columns (32 e4m3 / 64 bf16 bytes each, the
    // same bytes as the K-major slot), and fragments are read with ds_read_b64_tr_b8 / _b16, which hand
    // each lane consecutive K of one column.  A half-wave's transposing read covers 8 (e4m3) / 4 (bf16)
    // consecutive K rows in one contiguous 256-byte span, so the rows need no swizzle.
    static_assert(!BMN || (NB == 1 && (KIND == kFP8FP8 || KIND == kBF16)), "MN-major B: e4m3 / bf16, 32-column strips");
    constexpr int MN_E = kBf16 ? 2 : 1, MN_PITCH = 32 * MN_E;
    constexpr int SLOTB = BN * RG;                          // B part of a group slot
    constexpr int SLOT = SLOTB + AR * RGA;                  // bytes of one group slot
    constexpr int NBLK = NB * MT;                           // 32x32 output blocks
    constexpr int kLoads = kShape.loads;
    static_assert(kLoads == NDMA + NDMAA + (kBf16 ? 0 : G * (NB + MT)), "loads per group");
    static_assert(D >= 2 && (D - 1) * kLoads <= 63, "vmcnt range");
    constexpr int RING = NW * D * SLOT, RED = NW * NBLK * 4096;
    static_assert(RING <= 160 * 1024 && RED <= 128 * 1024, "LDS budget");
    // the wave rings, reused for the wave reduction after the main loop
    __shared__ __attribute__((aligned(1024))) uint8_t smem[RING > RED ? RING : RED];
    f32x4* const red = reinterpret_cast<f32x4*>(smem);

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int r = lane & 31, q = lane >> 5;

    // ------------------------------------------------------------------ strip and K range
    const int split_k = p.split_k;
    int t, split = 0;
    if (split_k > 1) {
        // grid = 8 * ceil(strips / 8) * split_k; all splits of a strip share blockIdx % 8 (XCD)
        const int b = vb, rr = b >> 3;
        t = (rr / split_k) * 8 + (b & 7);
        split = rr % split_k;
        if (p.split_spread) {
            // (test knob: consecutive workgroups -- different XCDs -- take the splits of a strip)
            t = b / split_k;
            split = b % split_k;
        }
        if (!BMN && t >= p.num_tiles) return;
    } else {
        t = vb;
    }
    if constexpr (BMN) {
        // The L = 128 / MN_PITCH strips whose K rows share 128-byte lines run on one XCD (workgroup t
        // runs on XCD t % 8; the host pads the grid to whole blocks of 8 L), so each line reaches one L2.
        constexpr int L = 128 / MN_PITCH;
        const int i = t % (8 * L);
        t = t - i + (i % 8) * L + i / 8;
        if (t >= p.num_tiles) return;
    }
    const int tile_id = t;
    const int nn = p.num_n_blocks;
    int batch = 0;
    if (p.gemm_type == kBatched || p.gemm_type == kMasked) {
        batch = t / nn;
        t -= batch * nn;
    }
    const int n0 = t * BN;
    const int N = p.n;
    // Masked groups hold masked_m[g] <= max_m valid rows (rows past them are neither read nor
    // written); an empty group's strips return at once (all its splits alike, so the split-K
    // arrival counts stay consistent).
    const int M = __builtin_amdgcn_readfirstlane(p.gemm_type == kMasked ? min(p.m, p.layout[batch]) : p.m);
    if (M <= 0) return;
    const uint8_t* a_base = p.a;
    const uint8_t* b_base = p.b + (BMN ? (int64_t)n0 * MN_E : (int64_t)n0 * p.ldb);
    const uint16_t* sfa = p.sfa;
    const uint16_t* sfb = p.sfb;
    uint8_t* d_base = p.d;
    if (p.gemm_type == kBatched || p.gemm_type == kMasked) {
        a_base += (int64_t)batch * p.bsa;
        b_base += (int64_t)batch * p.bsb;
        d_base += (int64_t)batch * p.bsd * p.out_esize;
        if (!kBf16) {
            sfa += (int64_t)batch * p.sfa_bs;
            sfb += (int64_t)batch * p.sfb_bs;
        }
    }
    const int rows_a = min(BM, M), rows_b = min(BN, N - n0);
    const int nk64 = ceil_div(p.k, 64);
    const int kb0 = split * p.split_stages;
    const int kb1 = split_k > 1 ? min(nk64, kb0 + p.split_stages) : nk64;
    // The workgroup's groups are dealt to its waves in contiguous runs (measured: contiguous
    // per-wave K ranges stream long rows faster than groups interleaved over the waves).
    const int ng = ceil_div(max(kb1 - kb0, 0), G);                 // groups of the workgroup
    const int gpw = ceil_div(ng, NW);
    const int gw0 = w * gpw;                                        // first group of this wave
    const int ngw = max(0, min(ng, gw0 + gpw) - gw0);               // groups of this wave

    const __amdgpu_buffer_rsrc_t rs_a = make_rsrc(a_base, (int64_t)rows_a * p.lda);
    const __amdgpu_buffer_rsrc_t rs_b =
        make_rsrc(b_base, BMN ? (int64_t)p.k * p.ldb - (int64_t)n0 * MN_E : (int64_t)rows_b * p.ldb);
    __amdgpu_buffer_rsrc_t rs_sa, rs_sb;
    if constexpr (!kBf16) {
        rs_sa = make_rsrc(sfa, (int64_t)nk64 * p.sfa_ld * 2);
        rs_sb = make_rsrc(sfb + n0, ((int64_t)nk64 * p.sfb_ld - n0) * 2);
    }
    // Per-lane row offsets (rows past the operand read zeros) and scale-dword offsets: the packed
    // scales of rows 2i and 2i + 1 share one dword (the leading dimension is even), so a lane
    // loads the aligned dword of its row pair and shifts its byte ((row % 2) * 2 + q) down at
    // use; the MFMA reads the low byte of the scale register.  (Byte loads would need a
    // zero-extension that the compiler hoists to the top of the loop, which makes it wait for
    // the ring's loads in flight.)
    uint32_t vsa[MT], vsb[NB];
    const int sc_shift = 8 * ((r & 1) * 2 + q);
#pragma unroll
    for (int jm = 0; jm < MT; ++jm) {
        const int row = jm * 32 + r;
        vsa[jm] = row < rows_a ? (uint32_t)((row & ~1) * 2) : kOOBOffset;
    }
#pragma unroll
    for (int jn = 0; jn < NB; ++jn) {
        const int row = jn * 32 + r;
        vsb[jn] = row < rows_b ? (uint32_t)((row & ~1) * 2) : kOOBOffset;
    }
    // B load instruction i of a group: lane l fills LDS slot l % SPR of row i RPI + l / SPR with
    // the row's 16-byte piece (slot ^ swizzle(row)) of the group.
    int lk[NDMA];
#pragma unroll
    for (int i = 0; i < NDMA; ++i) {
        const int row = i * RPI + lane / SPR;
        lk[i] = ((lane % SPR) ^ slot_swizzle<SPR>(row)) * 16;
    }
    uint32_t vrow[NDMA];   // (rows past the strip's end: out of range, zeros)
#pragma unroll
    for (int i = 0; i < NDMA; ++i) {
        const int row = i * RPI + lane / SPR;
        vrow[i] = row < rows_b ? (uint32_t)(row * p.ldb + lk[i]) : kOOBOffset;
    }
    // MN-major B: load instruction i fills LDS bytes [1024 i, +1024) of the slot's B part, i.e. K row
    // kr = (1024 i + 16 lane) / MN_PITCH of the group, column bytes (16 lane) % MN_PITCH (past the
    // strip's columns: out of range); lk[i] holds kr
    if constexpr (BMN) {
#pragma unroll
        for (int i = 0; i < NDMA; ++i) {
            const int o = i * 1024 + lane * 16;
            lk[i] = o / MN_PITCH;
            vrow[i] = (o % MN_PITCH) < rows_b * MN_E ? (uint32_t)(lk[i] * p.ldb + o % MN_PITCH) : kOOBOffset;
        }
    }
    int lka[NDMAA];
    uint32_t vrowa[NDMAA];
#pragma unroll
    for (int i = 0; i < NDMAA; ++i) {
        const int row = i * RPIA + lane / SPRA;
        lka[i] = ((lane % SPRA) ^ slot_swizzle<SPRA>(row)) * 16;
        vrowa[i] = row < rows_a ? (uint32_t)(row * p.lda + lka[i]) : kOOBOffset;
    }
    uint8_t* const ring = smem + w * (D * SLOT);
    const int kbytes_a = p.kbytes_a, kbytes_b = p.kbytes_b;
    const int sfa_step = (int)p.sfa_ld * 2, sfb_step = (int)p.sfb_ld * 2;

    // ------------------------------------------------------------------ register ring
    int sa[D][G][MT], sb[D][G][NB];
    // Group gi of this wave (64-K blocks kb0 + (gw0 + gi) G + j) into ring slot S; a group past
    // the wave's range (or a block past K) loads zeros with no memory traffic.
    auto load_group = [&](auto slot_tag, int gi) {
        constexpr int S = decltype(slot_tag)::value;
        const bool live = gi < ngw;
        const int kbg = kb0 + (gw0 + gi) * G;
        if constexpr (BMN) {
            // K rows of the group (rows past K or past the split's range read zeros)
            const int krows = live && kbg < kb1 ? min(p.k, kb1 * 64) - kbg * 64 : 0;
            const uint32_t kofs = (uint32_t)(kbg * 64) * (uint32_t)p.ldb;
#pragma unroll
            for (int i = 0; i < NDMA; ++i) {
                const uint32_t v = lk[i] < krows && vrow[i] != kOOBOffset ? vrow[i] + kofs : kOOBOffset;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rs_b, (lds_void*)(ring + S * SLOT + i * 1024), 16, v, 0, 0, 0);
            }
        } else {
            // B rows of the group: whole lines into the wave's ring slot S (a piece past K or past
            // the strip's rows reads zeros)
            const int left = live && kbg < kb1 ? kbytes_b - kbg * RBB : 0;
            const int kend = (kb1 - kbg) * RBB;   // (a group straddling the split's end stops there)
#pragma unroll
            for (int i = 0; i < NDMA; ++i) {
                const uint32_t v = lk[i] < left && lk[i] < kend ? vrow[i] : kOOBOffset;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rs_b, (lds_void*)(ring + S * SLOT + i * 1024), 16, v,
                                                         __builtin_amdgcn_readfirstlane(kbg * RBB), 0, 0);
            }
        }
        {
            // A rows likewise, behind the B rows of the slot
            const int left_a = live && kbg < kb1 ? kbytes_a - kbg * RBA : 0;
            const int kend_a = (kb1 - kbg) * RBA;
#pragma unroll
            for (int i = 0; i < NDMAA; ++i) {
                const uint32_t v = lka[i] < left_a && lka[i] < kend_a ? vrowa[i] : kOOBOffset;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rs_a, (lds_void*)(ring + S * SLOT + SLOTB + i * 1024), 16, v,
                                                         __builtin_amdgcn_readfirstlane(kbg * RBA), 0, 0);
            }
        }
        static_for<G>([&](auto j_c) {
            constexpr int j = decltype(j_c)::value;
            const int kb = kbg + j;
            const bool on = live && kb < kb1;
            if constexpr (!kBf16) {
#pragma unroll
                for (int jm = 0; jm < MT; ++jm)
                    sa[S][j][jm] = (int)__builtin_amdgcn_raw_buffer_load_b32(rs_sa, on ? vsa[jm] : kOOBOffset, kb * sfa_step, 0);
#pragma unroll
                for (int jn = 0; jn < NB; ++jn)
                    sb[S][j][jn] = (int)__builtin_amdgcn_raw_buffer_load_b32(rs_sb, on ? vsb[jn] : kOOBOffset, kb * sfb_step, 0);
            }
        });
    };

    f32x16 acc[NB][MT];
#pragma unroll
    for (int jn = 0; jn < NB; ++jn)
#pragma unroll
        for (int jm = 0; jm < MT; ++jm) acc[jn][jm] = f32x16{};

    // B fragment piece P of block j, strip block jn, from ring slot S
    auto b_piece = [&](int S, int j, int jn, int P) -> i32x4 {
        if constexpr (BMN) {
            // two transposing reads: lane (r, q) gets K [32 P + 16 q, +16) (e4m3) / [16 P + 8 q, +8) (bf16)
            // of column r of block j (the K-major piece's bytes).  e4m3: in each 16-lane group lane s
            // supplies the 8 bytes of K row k0 + s / 2 at column bytes 16 h + 8 (s % 2), and lane i
            // receives K k0 .. k0 + 7 of column 16 h + i; bf16: lane s supplies K row k0 + s / 4 at
            // columns 16 h + 4 (s % 4), and lane i receives K k0 .. k0 + 3 of column 16 h + i.
            typedef int v2i __attribute__((ext_vector_type(2)));
            const int s16 = lane & 15, h = (lane >> 4) & 1;
            const uint8_t* slot0 = ring + S * SLOT;
            if constexpr (!kBf16) {
                typedef __attribute__((address_space(3))) v2i lds_v2i;
                const uint8_t* b0 = slot0 + (j * 64 + 32 * P + 16 * q + (s16 >> 1)) * MN_PITCH + 16 * h + (s16 & 1) * 8;
                const v2i e0 = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i*)(b0));
                const v2i e1 = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i*)(b0 + 8 * MN_PITCH));
                return i32x4{e0[0], e0[1], e1[0], e1[1]};
            } else {
                typedef short v4s __attribute__((ext_vector_type(4)));
                typedef __attribute__((address_space(3))) v4s lds_v4s;
                const uint8_t* b0 = slot0 + (j * 64 + 16 * P + 8 * q + (s16 >> 2)) * MN_PITCH + 32 * h + (s16 & 3) * 8;
                const v2i e0 = __builtin_bit_cast(v2i, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)(b0)));
                const v2i e1 = __builtin_bit_cast(v2i, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)(b0 + 4 * MN_PITCH)));
                return i32x4{e0[0], e0[1], e1[0], e1[1]};
            }
        }
        const int R = jn * 32 + r;
        const int slot = (j * RBB + 32 * P) / 16 + q;
        return *reinterpret_cast<const i32x4*>(ring + S * SLOT + R * RG + ((slot ^ slot_swizzle<SPR>(R)) << 4));
    };
    // A fragment piece P of block j, tile block jm (rows past AR: zeros)
    auto a_piece = [&](int S, int j, int jm, int P) -> i32x4 {
        const int R = jm * 32 + r;
        const int Rc = R < AR ? R : AR - 1;
        const int slot = (j * RBA + 32 * P) / 16 + q;
        const i32x4 v = *reinterpret_cast<const i32x4*>(ring + S * SLOT + SLOTB + Rc * RGA +
                                                        ((slot ^ slot_swizzle<SPRA>(Rc)) << 4));
        return R < AR ? v : i32x4{0, 0, 0, 0};
    };
    auto compute = [&](auto slot_tag) {
        constexpr int S = decltype(slot_tag)::value;
        // this slot's loads are the oldest D - 1 groups back (the ring's LDS writes are not
        // visible to the compiler's own wait counting; the memory clobber keeps the LDS reads
        // below)
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"((D - 1) * kLoads) : "memory");
        i32x4 fb[G][NB][PB];
#pragma unroll
        for (int j = 0; j < G; ++j)
#pragma unroll
            for (int jn = 0; jn < NB; ++jn)
#pragma unroll
                for (int P = 0; P < PB; ++P) fb[j][jn][P] = b_piece(S, j, jn, P);
        i32x4 fa[G][MT][PA];
#pragma unroll
        for (int j = 0; j < G; ++j)
#pragma unroll
            for (int jm = 0; jm < MT; ++jm)
#pragma unroll
                for (int P = 0; P < PA; ++P) fa[j][jm][P] = a_piece(S, j, jm, P);
        static_for<G>([&](auto j_c) {
            constexpr int j = decltype(j_c)::value;
#pragma unroll
            for (int jn = 0; jn < NB; ++jn)
#pragma unroll
                for (int jm = 0; jm < MT; ++jm) {
                    if constexpr (kBf16) {
#pragma unroll
                        for (int s = 0; s < 4; ++s)
                            acc[jn][jm] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                                __builtin_bit_cast(bf16x8, fb[j][jn][s]), __builtin_bit_cast(bf16x8, fa[j][jm][s]),
                                acc[jn][jm], 0, 0, 0);
                    } else {
                        const i32x4 b0 = fb[j][jn][0], a0 = fa[j][jm][0];
                        i32x4 b1 = {0, 0, 0, 0}, a1 = {0, 0, 0, 0};
                        if constexpr (PB > 1) b1 = fb[j][jn][1];
                        if constexpr (PA > 1) a1 = fa[j][jm][1];
                        const i32x8 bf = {b0[0], b0[1], b0[2], b0[3], b1[0], b1[1], b1[2], b1[3]};
                        const i32x8 af = {a0[0], a0[1], a0[2], a0[3], a1[0], a1[1], a1[2], a1[3]};
                        acc[jn][jm] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
                            bf, af, acc[jn][jm], kFmtB, kFmtA, 0, shift_at_use(sb[S][j][jn], sc_shift), 0,
                            shift_at_use(sa[S][j][jm], sc_shift));
                    }
                }
        });
    };

    // ------------------------------------------------------------------ main loop
    // (groups issued in ring order, as in the loop, so that the compiler's wait counts at the loop
    // head see the same load order from both predecessors)
    static_for<D - 1>([&](auto s) {
        load_group(s, decltype(s)::value);
        __builtin_amdgcn_sched_barrier(0);
    });
    for (int i = 0; i < ngw; i += D) {
        static_for<D>([&](auto s_c) {
            constexpr int s = decltype(s_c)::value;
            load_group(Int<(s + D - 1) % D>{}, i + s + D - 1);
            __builtin_amdgcn_sched_barrier(0);
            compute(Int<s>{});   // (a group past the wave's range holds zeros: adds nothing)
            __builtin_amdgcn_sched_barrier(0);
        });
    }

    // ------------------------------------------------------------------ wave reduction
    // red[((w * NBLK + blk) * 4 + g) * 64 + lane] = elements 4 g .. 4 g + 3 of the wave's block,
    // over the rings once every wave is done with them (loads past a wave's range may still be
    // landing in its ring: wait for them first).
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
#pragma unroll
    for (int jn = 0; jn < NB; ++jn)
#pragma unroll
        for (int jm = 0; jm < MT; ++jm)
#pragma unroll
            for (int g = 0; g < 4; ++g)
                red[((w * NBLK + jn * MT + jm) * 4 + g) * 64 + lane] =
                    f32x4{acc[jn][jm][4 * g], acc[jn][jm][4 * g + 1], acc[jn][jm][4 * g + 2], acc[jn][jm][4 * g + 3]};
    __syncthreads();
    // Block blk is summed (waves in order) and finished by wave blk % NW.
    f32x16 out[NB][MT];
#pragma unroll
    for (int jn = 0; jn < NB; ++jn)
#pragma unroll
        for (int jm = 0; jm < MT; ++jm) {
            out[jn][jm] = f32x16{};
            if ((jn * MT + jm) % NW != w) continue;
            for (int ww = 0; ww < NW; ++ww)
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const f32x4 v = red[((ww * NBLK + jn * MT + jm) * 4 + g) * 64 + lane];
#pragma unroll
                    for (int i = 0; i < 4; ++i) out[jn][jm][4 * g + i] += v[i];
                }
        }

    // ------------------------------------------------------------------ split-K across workgroups
    if (split_k > 1) {
        // Partials in accumulator-register order; lanes of rows past M take an offset past the
        // buffer's end (no bytes move for them).
        float* const tile_ws = p.ws + (int64_t)tile_id * split_k * (NBLK * 1024);
        const __amdgpu_buffer_rsrc_t rs_ws = make_rsrc(tile_ws, (int64_t)split_k * NBLK * 1024 * 4);
        auto part_off = [&](int sp, int blk, int jm) -> uint32_t {
            return jm * 32 + r < M ? (uint32_t)((sp * NBLK + blk) * 1024 + lane * 16) * 4u : kOOBOffset;
        };
#pragma unroll
        for (int jn = 0; jn < NB; ++jn)
#pragma unroll
            for (int jm = 0; jm < MT; ++jm) {
                if ((jn * MT + jm) % NW != w) continue;
                const uint32_t off = part_off(split, jn * MT + jm, jm);
#pragma unroll
                for (int g = 0; g < 4; ++g)
                    __builtin_amdgcn_raw_buffer_store_b128(
                        __builtin_bit_cast(u32x4, f32x4{out[jn][jm][4 * g], out[jn][jm][4 * g + 1], out[jn][jm][4 * g + 2],
                                                        out[jn][jm][4 * g + 3]}),
                        rs_ws, off + 16 * g, 0, kCacheSc1);
            }
        // Arrival count.  The partials were stored at device scope, so once every wave's stores
        // are acknowledged they are visible on every XCD; no fence (which would write back or
        // invalidate the whole L2) is needed on either side.  This follows the GFX942 code
        // sequences of the LLVM AMDGPU memory model (llvm/docs/AMDGPUUsage.rst, "Memory Model
        // GFX942", which gfx950 shares): a monotonic agent-scope atomic store or load is a plain
        // buffer store / load with sc1 set, so the partial stores and loads here are relaxed
        // agent-scope atomics; a release at agent scope is "buffer_wbl2 sc1=1; s_waitcnt vmcnt(0)",
        // where the L2 writeback serves only non-atomic data, so for these stores the vmcnt(0)
        // before the counter's fetch-add is the whole release; an acquire is "buffer_inv sc1=1"
        // after the atomic, which again serves only non-atomic loads, so the sc1 loads of the
        // last workgroup need no invalidate.  (tests/test_split_k_gpu.py forces the splits of
        // one tile onto different XCDs to keep this checked.)
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        int* flag = reinterpret_cast<int*>(red);
        if (tid == 0)
            *flag = __hip_atomic_fetch_add(p.counters + tile_id, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __syncthreads();
        const int prev = *flag;
        if (prev != split_k - 1) return;
#pragma unroll
        for (int jn = 0; jn < NB; ++jn)
#pragma unroll
            for (int jm = 0; jm < MT; ++jm) {
                if ((jn * MT + jm) % NW != w) continue;
                out[jn][jm] = f32x16{};
                for (int sp = 0; sp < split_k; ++sp) {
                    const uint32_t off = part_off(sp, jn * MT + jm, jm);
#pragma unroll
                    for (int g = 0; g < 4; ++g) {
                        const f32x4 v = __builtin_bit_cast(
                            f32x4, __builtin_amdgcn_raw_buffer_load_b128(rs_ws, off + 16 * g, 0, kCacheSc1));
#pragma unroll
                        for (int i = 0; i < 4; ++i) out[jn][jm][4 * g + i] += v[i];
                    }
                }
            }
        if (tid == 0) __hip_atomic_store(p.counters + tile_id, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }

    // ------------------------------------------------------------------ epilogue
#pragma unroll
    for (int jn = 0; jn < NB; ++jn)
#pragma unroll
        for (int jm = 0; jm < MT; ++jm) {
            if ((jn * MT + jm) % NW != w) continue;
            const int m = jm * 32 + r;
            epilogue_block<EPI>(p, out[jn][jm], d_base, m, m < M, false, n0 + jn * 32, N, batch, q);
        }
}

}  // namespace dg


namespace dg {

// Decode kernel with one shared ring.  The tile is 32 MT x 32 NB like skinny_kernel's (a dense or
// batched M above 32 MT takes several tiles per strip), but its NW = MT x NB waves split the tile
// instead of K: wave w owns the 32x32 output block
// (w % MT, w / MT) over the workgroup's whole K range.  All waves walk the same groups of G 64-K
// blocks through one ring of D group slots (B rows of the strip, all 32 MT rows of A, and the
// packed scale rows of both) that they fill together, so every byte is fetched once per
// workgroup, the ring keeps D - 1 groups in flight, and no wave reduction is needed at the end.
// One workgroup barrier per group certifies that the group has landed (every wave waited for its
// own share of the loads) and that the slot it refills was read by every wave.  Every load of the
// loop goes global -> LDS, so no vector-memory result lands in a register and the only waits are
// the explicit per-group ones.
template <int KIND, int MT, int NB, int D, int EPI>
__device__ __forceinline__ void skinny_rows_body(const KParams& p, const int vb) {
    constexpr bool kAFp4 = KIND == kFP4FP4;
    constexpr bool kBFp4 = KIND == kFP8FP4 || KIND == kFP4FP4;
    constexpr bool kBf16 = KIND == kBF16;
    constexpr int kFmtA = kAFp4 ? kFmtE2M1 : kFmtE4M3;
    constexpr int kFmtB = kBFp4 ? kFmtE2M1 : kFmtE4M3;
    constexpr int NW = MT * NB;
    constexpr int BM = 32 * MT, BN = 32 * NB;
    static_assert(BM <= 128 && BN <= 128, "one scale dword per lane covers 128 rows");
    constexpr int RBA = kBf16 ? 128 : (kAFp4 ? 32 : 64);   // bytes of one row per 64-K block
    constexpr int RBB = kBf16 ? 128 : (kBFp4 ? 32 : 64);
    constexpr int PA = RBA / 32, PB = RBB / 32;            // 16-byte pieces per lane and block
    constexpr SkinnyShape kShape = skinny_shape(KIND, MT, NB, BM);
    constexpr int G = kShape.g, RG = kShape.rg, RGA = kShape.rga;
    constexpr int SPR = RG / 16, SPRA = RGA / 16;           // 16-byte slots of a B / A row
    constexpr int RPI = 64 / SPR, RPIA = 64 / SPRA;         // rows per load instruction
    constexpr int NDMA = BN / RPI, NDMAA = BM / RPIA;       // row-load instructions per group slot
    constexpr int NLR = NDMA + NDMAA;
    constexpr int NSF = kBf16 ? 0 : 2 * G;                  // scale-row loads per group (A, B per 64-K block)
    constexpr int LPR = (NLR + NW - 1) / NW;                // row loads per wave and group
    constexpr int LPS = (NSF + NW - 1) / NW;                // scale loads per wave and group
    constexpr int PG = LPR + LPS;                           // vector-memory instructions per wave and group
    constexpr int SLOTB = BN * RG;
    constexpr int SCOFF = SLOTB + BM * RGA;                 // scale rows: A blocks, then B blocks, 256 B each
    constexpr int SLOT = SCOFF + NSF * 256;
    constexpr int SPARE = (NLR % NW != 0 || NSF % NW != 0) ? 1024 : 0;   // lands dead loads
    static_assert(BM % RPIA == 0 && BN % RPI == 0, "slot rows");
    static_assert(D >= 3 && (D - 2) * PG <= 63, "vmcnt range");
    static_assert(D * SLOT + SPARE <= 160 * 1024, "LDS budget");
    __shared__ __attribute__((aligned(1024))) uint8_t smem[D * SLOT + SPARE];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wjm = w % MT, wjn = w / MT;
    const int r = lane & 31, q = lane >> 5;

    // ------------------------------------------------------------------ strip and K range
    const int split_k = p.split_k;
    int t, split = 0;
    if (split_k > 1) {
        // grid = 8 * ceil(strips / 8) * split_k; all splits of a strip share blockIdx % 8 (XCD)
        const int b = vb, rr = b >> 3;
        t = (rr / split_k) * 8 + (b & 7);
        split = rr % split_k;
        if (p.split_spread) {
            t = b / split_k;
            split = b % split_k;
        }
        if (t >= p.num_tiles) return;
    } else {
        t = vb;
    }
    const int tile_id = t;
    // tile = (batch, strip, M block).  With M in several row blocks (dense and batched launches whose M
    // exceeds the BM rows of one tile; masked launches have one) the strips are padded to whole groups of
    // eight and a strip's row blocks are tile ids eight apart, on one XCD, so its L2 fetches the strip's B
    // rows once; tiles of padding strips exit.
    const int nn = p.num_n_blocks, nmb = p.num_m_blocks;
    const int nnp = nmb > 1 ? (nn + 7) / 8 * 8 : nn;
    int batch = 0;
    if (p.gemm_type == kBatched || p.gemm_type == kMasked) {
        batch = t / (nnp * nmb);
        t -= batch * (nnp * nmb);
    }
    const int m0 = nmb > 1 ? ((t >> 3) % nmb) * BM : 0;
    if (nmb > 1) t = (t >> 3) / nmb * 8 + (t & 7);
    if (t >= nn) return;
    const int n0 = t * BN;
    const int N = p.n;
    const int M = __builtin_amdgcn_readfirstlane(p.gemm_type == kMasked ? min(p.m, p.layout[batch]) : p.m);
    if (M <= m0) return;
    const uint8_t* a_base = p.a + (int64_t)m0 * p.lda;
    const uint8_t* b_base = p.b + (int64_t)n0 * p.ldb;
    const uint16_t* sfa = p.sfa + m0;
    const uint16_t* sfb = p.sfb;
    uint8_t* d_base = p.d;
    if (p.gemm_type == kBatched || p.gemm_type == kMasked) {
        a_base += (int64_t)batch * p.bsa;
        b_base += (int64_t)batch * p.bsb;
        d_base += (int64_t)batch * p.bsd * p.out_esize;
        if (!kBf16) {
            sfa += (int64_t)batch * p.sfa_bs;
            sfb += (int64_t)batch * p.sfb_bs;
        }
    }
    const int rows_a = min(BM, M - m0), rows_b = min(BN, N - n0);
    const int nk64 = ceil_div(p.k, 64);
    const int kb0 = split * p.split_stages;
    const int kb1 = split_k > 1 ? min(nk64, kb0 + p.split_stages) : nk64;
    const int ng = ceil_div(max(kb1 - kb0, 0), G);   // groups of the workgroup (every wave walks all)
    const int kbytes_a = p.kbytes_a, kbytes_b = p.kbytes_b;

    // Row loads: the group's NLR instructions are dealt to the waves (wave w issues w, w + NW, ...);
    // instruction i < NDMA fills B rows [i RPI, +RPI) of the slot, the others A rows.  Everything
    // wave-uniform about load j (its tensor, LDS offset, row bytes per 64-K block, K row bytes) is
    // fixed here; a load past NLR is dead (out of range, into the spare kilobyte).
    // (arrays or conditional expressions of buffer-resource type lose the kernel's host stub, so
    // each load keeps its tensor's base and size and builds the resource at issue)
    const uint8_t* ld_base[LPR];
    int64_t ld_size[LPR];
    int ld_lds[LPR], ld_rb[LPR], ld_kb[LPR], ld_lk[LPR];
    uint32_t ld_v[LPR];
#pragma unroll
    for (int j = 0; j < LPR; ++j) {
        const int i = w + j * NW;
        const bool is_a = i >= NDMA;
        ld_base[j] = is_a ? a_base : b_base;
        ld_size[j] = is_a ? (int64_t)rows_a * p.lda : (int64_t)rows_b * p.ldb;
        ld_rb[j] = is_a ? RBA : RBB;
        ld_kb[j] = i < NLR ? (is_a ? kbytes_a : kbytes_b) : 0;
        const int spr = is_a ? SPRA : SPR;
        const int row = (is_a ? (i - NDMA) * RPIA : i * RPI) + lane / spr;
        const int sw = is_a ? slot_swizzle<SPRA>(row) : slot_swizzle<SPR>(row);
        ld_lk[j] = ((lane % spr) ^ sw) * 16;
        const bool row_ok = row < (is_a ? rows_a : rows_b);
        ld_v[j] = i < NLR && row_ok ? (uint32_t)(row * (is_a ? p.lda : p.ldb) + ld_lk[j]) : kOOBOffset;
        ld_lds[j] = i >= NLR ? D * SLOT : (is_a ? SLOTB + (i - NDMA) * 1024 : i * 1024);
    }
    // Scale loads: load j of this wave is scale row s = w + j NW of the group (s < G: A's packed
    // int16 pairs of 64-K block s, else B's of block s - G), one dword = two rows per lane.
    const uint16_t* sc_base[LPS > 0 ? LPS : 1];
    int64_t sc_size[LPS > 0 ? LPS : 1];
    int sc_lds[LPS > 0 ? LPS : 1], sc_blk[LPS > 0 ? LPS : 1], sc_step[LPS > 0 ? LPS : 1];
    uint32_t sc_v[LPS > 0 ? LPS : 1];
    if constexpr (LPS > 0) {
#pragma unroll
        for (int j = 0; j < LPS; ++j) {
            const int s = w + j * NW;
            const bool is_a = s < G;
            sc_base[j] = is_a ? sfa : sfb + n0;
            sc_size[j] = is_a ? ((int64_t)nk64 * p.sfa_ld - m0) * 2 : ((int64_t)nk64 * p.sfb_ld - n0) * 2;
            sc_step[j] = (int)(is_a ? p.sfa_ld : p.sfb_ld) * 2;
            sc_blk[j] = is_a ? s : s - G;
            sc_v[j] = s < NSF && 2 * lane < (is_a ? rows_a : rows_b) ? (uint32_t)(lane * 4) : kOOBOffset;
            sc_lds[j] = s < NSF ? SCOFF + s * 256 : D * SLOT;
        }
    }

    // Group gi (64-K blocks kb0 + gi G + j) into ring slot `slot`; a group past the range (or a
    // piece past K or past the split's end) loads zeros with no memory traffic.
    auto load_group = [&](int slot, int gi) {
        const bool live = gi < ng;
        const int kbg = kb0 + gi * G;
        uint8_t* const sbase = smem + slot * SLOT;
#pragma unroll
        for (int j = 0; j < LPR; ++j) {
            const int left = live ? ld_kb[j] - kbg * ld_rb[j] : 0;
            const int kend = (kb1 - kbg) * ld_rb[j];
            const uint32_t v = ld_lk[j] < left && ld_lk[j] < kend ? ld_v[j] : kOOBOffset;
            uint8_t* dst = ld_lds[j] >= D * SLOT ? smem + D * SLOT : sbase + ld_lds[j];
            __builtin_amdgcn_raw_ptr_buffer_load_lds(make_rsrc(ld_base[j], ld_size[j]), (lds_void*)dst, 16, v,
                                                     __builtin_amdgcn_readfirstlane(kbg * ld_rb[j]), 0, 0);
        }
        if constexpr (LPS > 0) {
#pragma unroll
            for (int j = 0; j < LPS; ++j) {
                const int kb = kbg + sc_blk[j];
                const bool on = live && kb < kb1;
                uint8_t* dst = sc_lds[j] >= D * SLOT ? smem + D * SLOT : sbase + sc_lds[j];
                __builtin_amdgcn_raw_ptr_buffer_load_lds(make_rsrc(sc_base[j], sc_size[j]), (lds_void*)dst, 4,
                                                         on ? sc_v[j] : kOOBOffset,
                                                         __builtin_amdgcn_readfirstlane(on ? kb * sc_step[j] : 0), 0, 0);
            }
        }
    };

    f32x16 acc = f32x16{};
    const int RBr = wjn * 32 + r, RAr = wjm * 32 + r;
    auto compute = [&](int slot) {
        const uint8_t* sb_ = smem + slot * SLOT;
        i32x4 fb[G][PB], fa[G][PA];
        int sca[G], scb[G];
#pragma unroll
        for (int j = 0; j < G; ++j) {
#pragma unroll
            for (int P = 0; P < PB; ++P) {
                const int sl = (j * RBB + 32 * P) / 16 + q;
                fb[j][P] = *reinterpret_cast<const i32x4*>(sb_ + RBr * RG + ((sl ^ slot_swizzle<SPR>(RBr)) << 4));
            }
#pragma unroll
            for (int P = 0; P < PA; ++P) {
                const int sl = (j * RBA + 32 * P) / 16 + q;
                fa[j][P] = *reinterpret_cast<const i32x4*>(sb_ + SLOTB + RAr * RGA + ((sl ^ slot_swizzle<SPRA>(RAr)) << 4));
            }
            if constexpr (!kBf16) {
                sca[j] = sb_[SCOFF + j * 256 + RAr * 2 + q];
                scb[j] = sb_[SCOFF + (G + j) * 256 + RBr * 2 + q];
            }
        }
        static_for<G>([&](auto j_c) {
            constexpr int j = decltype(j_c)::value;
            if constexpr (kBf16) {
#pragma unroll
                for (int s = 0; s < 4; ++s)
                    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, fb[j][s]),
                                                                  __builtin_bit_cast(bf16x8, fa[j][s]), acc, 0, 0, 0);
            } else {
                const i32x4 b0 = fb[j][0], a0 = fa[j][0];
                i32x4 b1 = {0, 0, 0, 0}, a1 = {0, 0, 0, 0};
                if constexpr (PB > 1) b1 = fb[j][1];
                if constexpr (PA > 1) a1 = fa[j][1];
                const i32x8 bf = {b0[0], b0[1], b0[2], b0[3], b1[0], b1[1], b1[2], b1[3]};
                const i32x8 af = {a0[0], a0[1], a0[2], a0[3], a1[0], a1[1], a1[2], a1[3]};
                acc = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(bf, af, acc, kFmtB, kFmtA, 0, scb[j], 0, sca[j]);
            }
        });
    };

    // ------------------------------------------------------------------ main loop
    // Groups 0 .. D-2 in flight; then per group g: wait for this wave's share of g, barrier (g is
    // complete in LDS and slot (g - 1) % D is read by every wave), refill that slot with group
    // g + D - 1, compute g.  The wait count holds because every wave issues exactly PG
    // vector-memory instructions per group, in group order.
    for (int g = 0; g < D - 1; ++g) load_group(g, g);
    int slot = 0;
    for (int g = 0; g < ng; ++g) {
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"((D - 2) * PG) : "memory");
        stage_barrier();
        load_group(slot == 0 ? D - 1 : slot - 1, g + D - 1);
        __builtin_amdgcn_sched_barrier(0);
        compute(slot);
        __builtin_amdgcn_sched_barrier(0);
        slot = slot + 1 == D ? 0 : slot + 1;
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

    const int m = m0 + wjm * 32 + r;
    // ------------------------------------------------------------------ split-K across workgroups
    if (split_k > 1) {
        constexpr int NBLK = NW;
        float* const tile_ws = p.ws + (int64_t)tile_id * split_k * (NBLK * 1024);
        const __amdgpu_buffer_rsrc_t rs_ws = make_rsrc(tile_ws, (int64_t)split_k * NBLK * 1024 * 4);
        const int blk = wjn * MT + wjm;
        auto part_off = [&](int sp) -> uint32_t {
            return m < M ? (uint32_t)((sp * NBLK + blk) * 1024 + lane * 16) * 4u : kOOBOffset;
        };
        if (p.split_reduce) {
            // the second launch (split_reduce_kernel) sums the partials: plain stores, made visible
            // to it by the kernel boundary, and no arrival count
            const uint32_t off = part_off(split);
#pragma unroll
            for (int g = 0; g < 4; ++g)
                __builtin_amdgcn_raw_buffer_store_b128(
                    __builtin_bit_cast(u32x4, f32x4{acc[4 * g], acc[4 * g + 1], acc[4 * g + 2], acc[4 * g + 3]}), rs_ws,
                    off + 16 * g, 0, 0);
            return;
        }
        {
            const uint32_t off = part_off(split);
#pragma unroll
            for (int g = 0; g < 4; ++g)
                __builtin_amdgcn_raw_buffer_store_b128(
                    __builtin_bit_cast(u32x4, f32x4{acc[4 * g], acc[4 * g + 1], acc[4 * g + 2], acc[4 * g + 3]}), rs_ws,
                    off + 16 * g, 0, kCacheSc1);
        }
        // Arrival count: device-scope partial stores and loads, no fence (the memory-model argument
        // of skinny_kernel's split-K).
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        int* flag = reinterpret_cast<int*>(smem);
        if (tid == 0)
            *flag = __hip_atomic_fetch_add(p.counters + tile_id, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __syncthreads();
        if (*flag != split_k - 1) return;
        acc = f32x16{};
        for (int sp = 0; sp < split_k; ++sp) {
            const uint32_t off = part_off(sp);
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const f32x4 v =
                    __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rs_ws, off + 16 * g, 0, kCacheSc1));
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[4 * g + i] += v[i];
            }
        }
        if (tid == 0) __hip_atomic_store(p.counters + tile_id, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }

    // ------------------------------------------------------------------ epilogue
    epilogue_block<EPI>(p, acc, d_base, m, m < M, false, n0 + wjn * 32, N, batch, q);
}

// (the body lives in a device function: written directly in the kernel, clang's host pass at -O1
// and above emitted no launch stub for it)
template <int KIND, int MT, int NB, int D, int EPI>
__global__ __launch_bounds__(MT * NB * 64, 1) void skinny_rows_kernel(const KParams p) {
    skinny_rows_body<KIND, MT, NB, D, EPI>(p, blockIdx.x + p.vbase);
}

// Second launch of a split-K shared-ring plan (KParams::split_reduce): one wave per 32x32 output
// block (block b = waves per workgroup x workgroup + wave, over the tiles' MT x NB blocks in the
// first launch's order) sums the block's split_k fp32 partials in split order -- the same sums, in
// the same order, as the first launch's own last-arriving workgroup would form, so D is the same bit
// for bit -- and runs the block's epilogue.  The loads of up to eight splits are issued before any
// is added.  Spreading the reduction over one wave per block keeps it off the critical path of a
// single CU, whose load rate bounds how many partials one workgroup can sum quickly.
template <int MT, int NB, int EPI>
__device__ __forceinline__ void split_reduce_body(const KParams& p, const int vb) {
    constexpr int NBLK = MT * NB, BN = 32 * NB;
    constexpr int CH = 8;
    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int gb = vb * (int)(blockDim.x >> 6) + w;
    const int tile_id = gb / NBLK, blk = gb - tile_id * NBLK;
    if (tile_id >= p.num_tiles) return;
    const int wjm = blk % MT, wjn = blk / MT;
    const int r = lane & 31, q = lane >> 5;
    // (the first launch's tile numbering: strips padded to groups of eight when M takes several row blocks)
    const int nn = p.num_n_blocks, nmb = p.num_m_blocks;
    const int nnp = nmb > 1 ? (nn + 7) / 8 * 8 : nn;
    int t = tile_id, batch = 0;
    if (p.gemm_type == kBatched || p.gemm_type == kMasked) {
        batch = t / (nnp * nmb);
        t -= batch * (nnp * nmb);
    }
    const int m0 = nmb > 1 ? ((t >> 3) % nmb) * MT * 32 : 0;
    if (nmb > 1) t = (t >> 3) / nmb * 8 + (t & 7);
    if (t >= nn) return;
    const int M = __builtin_amdgcn_readfirstlane(p.gemm_type == kMasked ? min(p.m, p.layout[batch]) : p.m);
    if (M <= m0) return;
    uint8_t* d_base = p.d;
    if (p.gemm_type == kBatched || p.gemm_type == kMasked) d_base += (int64_t)batch * p.bsd * p.out_esize;
    const int m = m0 + wjm * 32 + r;
    const int split_k = p.split_k;
    const float* const tile_ws = p.ws + (int64_t)tile_id * split_k * (NBLK * 1024);
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(tile_ws, (int64_t)split_k * NBLK * 1024 * 4);
    const uint32_t off0 = m < M ? (uint32_t)(blk * 1024 + lane * 16) * 4u : kOOBOffset;
    f32x16 acc = f32x16{};
    for (int sp0 = 0; sp0 < split_k; sp0 += CH) {
        f32x4 v[CH][4];
#pragma unroll
        for (int j = 0; j < CH; ++j) {
            const uint32_t off = sp0 + j < split_k && off0 != kOOBOffset ? off0 + (uint32_t)(sp0 + j) * (NBLK * 4096u) : kOOBOffset;
#pragma unroll
            for (int g = 0; g < 4; ++g)
                v[j][g] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, off + 16 * g, 0, 0));
        }
        __builtin_amdgcn_sched_barrier(0);
        // (a split past the last adds -0.0, the exact identity of IEEE addition, so no add is
        // conditional and every load of the chunk is issued before the first add)
#pragma unroll
        for (int j = 0; j < CH; ++j) {
            const bool on = sp0 + j < split_k;
#pragma unroll
            for (int g = 0; g < 4; ++g)
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[4 * g + i] += on ? v[j][g][i] : -0.0f;
        }
    }
    epilogue_block<EPI>(p, acc, d_base, m, m < M, false, t * BN + wjn * 32, p.n, batch, q);
}

template <int MT, int NB, int EPI>
__global__ __launch_bounds__(256) void split_reduce_kernel(const KParams p) {
    split_reduce_body<MT, NB, EPI>(p, blockIdx.x + p.vbase);
}

template <int KIND, int MT, int NB, int NW, int D, int AR, int EPI, bool BMN = false>
__global__ __launch_bounds__(NW * 64, NW <= 4 ? 2 : 1) void skinny_kernel(const KParams p) {
    skinny_body<KIND, MT, NB, NW, D, AR, EPI, BMN>(p, blockIdx.x + p.vbase);
}

}  // namespace dg
