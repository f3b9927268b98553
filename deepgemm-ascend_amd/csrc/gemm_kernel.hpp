// Block-scaled GEMM kernel for gfx950 (MI355X).
//
// D = alpha * A . B^T (+ bias | + D) for K-major A [M,K] and B [N,K], with one UE8M0 scale
// per 32 K-elements and per row of each operand (the MX recipe of the reference's
// fp8_gemm_impl, deep_gemm/include/deep_gemm/fp8_gemm.hpp:36-287), computed on CDNA4
// v_mfma_scale_f32_32x32x64_f8f6f4 (e4m3 / e2m1 operands) or v_mfma_f32_32x32x16_bf16.
//
// One workgroup of NW = 4 or 8 waves (WGM x WGN over the BM x BN tile) walks K in stages of
// 64 (fp8 / fp4) or 32 (bf16) elements through an NSTAGE-deep ring of LDS stages:
//   HBM/L2 --buffer_load ... lds (operand rows and the packed-SF rows)--> LDS stage
//          --ds_read_b128--> VGPR fragments --MFMA--> fp32 accumulators (AGPRs)
//          --epilogue (alpha / bias / accumulate, RNE bf16) in registers--> D.
// Loads for stage c + NSTAGE - 1 are issued while stage c computes, so a stage has
// NSTAGE - 2 stages of compute to arrive.  A-side fragments (and scales) of stage c + 1 are
// read during stage c into a second register set, so the MFMAs never wait on their LDS
// reads except at a tile's first stage; B-side fragments stream one block ahead.  There is
// one workgroup barrier per stage.
//
// MFMA register layouts (measured on gfx950), lane l = r + 32 q (r = row 0..31, q = 0..1):
//   32x32x64 e4m3 operand: bytes [0,16) hold K [16q, 16q+16), bytes [16,32) hold K [32+16q, +16)
//   32x32x64 e2m1 operand: 16 bytes hold K [32q, 32q+32) (low nibble = even k)
//   scale operand of lane (r, q): UE8M0 exponent of K-block q (K [32q, 32q+32)) of row r
//   32x32x16 bf16 operand: 8 values hold K [8q, 8q+8)
//   accumulator: lane l, element i -> (row 4 (l/32) + (i%4) + 8 (i/4) of the MFMA "A" side,
//                column l%32)
// The kernel feeds B (n) as the MFMA "A" operand and A (m) as the "B" operand, so each lane
// ends with groups of four consecutive n of one output row m.
#pragma once

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
    int64_t sfa_ld, sfb_ld, sfa_bs, sfb_bs;   // int16 elements (ld even)
    int gemm_type, out_esize, accumulate, has_bias, alignment, vec_store;   // out_esize: bytes per D element
    float alpha;
    int num_m_blocks, num_n_blocks;
    int kbytes_a, kbytes_b;    // bytes of one K row (multiple of 16)
    int group_m;               // tile-order swizzle width along M
    // Split-K: the K loop of every tile is cut into split_k ranges of split_stages 64-K stages,
    // one workgroup each; the partial fp32 tiles meet in `ws` and the last workgroup of a tile
    // (per `counters`, which every launch leaves at zero) reduces them and runs the epilogue.
    int split_k, split_stages;
    int num_tiles;             // tiles of the launch (split-K grids are padded past it)
    float* ws;
    int* counters;
    int split_spread;          // test knob: the splits of a tile go to consecutive workgroups (other XCDs)
    int split_reduce;          // split-K partials summed by a second launch (split_reduce_kernel)
    // M-grouped psum GEMMs with tiles anchored at each group's first row (BM need not divide the
    // alignment): an upper bound of the tile count is launched; the grid's extra workgroups exit.
    int anchored;
    const int* runs;           // anchored m_indices GEMMs: the run table of the layout (m_indices_runs)
    // FP8 output: per-(row, 32 columns) UE8M0 exponents, packed in pairs into int16
    // sfd[(batch * n + col) / 64 * sfd_ld + row], lower byte = the even 32-column block.
    uint8_t* sfd;
    int64_t sfd_ld;
    // Persistent launches: bytes of each operand / SF tensor over all its batches or groups (every
    // span below 2^31, so a tile's base fits a buffer instruction's scalar offset).
    int64_t a_span, b_span, sfa_span, sfb_span;
    // Workgroups of the launch plan (vgrid) and the first one this launch serves (vbase): under a
    // CU cap (set_num_sms) the plan's workgroups go out in launches of at most that many, and
    // workgroup b of a launch serves plan workgroup vbase + b.
    int vgrid, vbase;
};

// Epilogue variants.
constexpr int kEpiF32 = 1;       // fp32 D (bias / accumulate allowed)
constexpr int kEpiBf16 = 2;      // bf16 D
constexpr int kEpiBf16SR = 3;    // bf16 D, stochastic rounding (no bias / accumulate / alpha)
constexpr int kEpiFp8 = 4;       // e4m3 D with per-(row, 32 columns) UE8M0 scales (n % 128 == 0)

// Stochastic rounding of four consecutive fp32 outputs of a row (columns 4j .. 4j+3) to bf16.
// The random bits come from a hash of the four fp32 bit patterns and the quartet index j
// (tests/utils.py:70-92 of the reference pins the exact function, with zeros standing in for
// columns past the end of the row): value v rounds up when its discarded low 16 bits exceed
// 0xffff minus its 16 random bits; NaN becomes the canonical 0x7fc0.
__device__ __forceinline__ void sr_bf16_quartet(const float* x, uint32_t j, uint16_t* out) {
    uint32_t v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = __builtin_bit_cast(uint32_t, x[i]);
    uint32_t h = v[0] * 0x5671d42bu + v[1] * 0x9995e499u + v[2] * 0xace1b8a5u + v[3] * 0xe153538du + j;
    h = (h ^ (h >> 23)) * 0x7feb352du;
    h ^= h >> 16;
    uint32_t h1 = h * 0x846ca68bu, h2 = h * 0xd35a2d97u;
    h1 ^= h1 >> 11;
    h2 ^= h2 >> 11;
    const uint32_t rnd[4] = {h1 & 0xffffu, h1 >> 16, h2 & 0xffffu, h2 >> 16};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t up = (v[i] & 0xffffu) > (0xffffu - rnd[i]) ? 1u : 0u;
        out[i] = (v[i] & 0x7fffffffu) > 0x7f800000u ? (uint16_t)0x7fc0 : (uint16_t)((v[i] >> 16) + up);
    }
}

// UE8M0 exponent s of the scale 2^(s-127) for a block whose largest magnitude has bf16 bits
// `x` (sign cleared): the smallest power of two with |max| <= 448 * 2^(s-127), at least 2^-22.
// With x = (e << 7) | mant, |max| / 448 <= 2^(e-8) exactly when mant <= 0x60 (448 = 1.75 * 2^8),
// so s = e - 8 + (mant > 0x60) = ((x + 31) >> 7) - 8; the floor of 2^-22 is the quantiser's
// clamp of the block maximum at 1e-4 (tests/generators.py:80-81 of the reference).
__device__ __forceinline__ uint32_t ue8m0_of_bf16_amax(uint32_t x) {
    return max((x + 31u) >> 7, 113u) - 8u;
}

template <int N>
struct Int { static constexpr int value = N; };

// Compile-time loop f(Int<0>), ..., f(Int<N-1>) (the kernel sources use no standard-library
// header, so the runtime compiler needs nothing beyond them).
template <int... Is>
struct IntSeq {};
template <int N, int... Is>
struct MakeSeq : MakeSeq<N - 1, N - 1, Is...> {};
template <int... Is>
struct MakeSeq<0, Is...> { using type = IntSeq<Is...>; };
template <typename F, int... Is>
__device__ __forceinline__ void static_for_impl(F&& f, IntSeq<Is...>) {
    (f(Int<Is>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
    static_for_impl(f, typename MakeSeq<N>::type{});
}

template <bool C, typename T, typename F>
struct Cond { using type = T; };
template <typename T, typename F>
struct Cond<false, T, F> { using type = F; };

template <typename A, typename B>
struct Pair {
    A first;
    B second;
};

// s_waitcnt that bounds only the vector-memory counter.
template <int VM>
__device__ __forceinline__ void wait_vmcnt() {
    constexpr int v = VM > 63 ? 63 : (VM < 0 ? 0 : VM);
    __builtin_amdgcn_s_waitcnt((v & 0xf) | ((v >> 4) << 14) | (0x7 << 4) | (0xf << 8));
}

// Slot swizzle inside one LDS row of SPR 16-byte slots (128-byte rows: 8 slots, 64-byte: 4,
// 32-byte: 2).  gfx950's LDS has 64 banks of 4 bytes and serves a ds_read_b128 in four phases
// of 16 lanes; measured (per-lane-pair bank-conflict counts), the phases of lanes 0..31 are
// {0-3, 12-15, 20-27} and {4-11, 16-19, 28-31} (lanes 32..63 alike).  With j = row / 4 those
// are the rows of even and of odd popcount(j % 8).  A phase is conflict-free when its 16 lanes
// (16 rows, one slot each) hit 16 distinct 16-byte bank groups of the 256-byte bank period:
//   64-byte rows:  row % 4 picks the quarter, so the slot must differ over the four j of each
//                  parity class: j % 4 does;
//   128-byte rows: row % 2 picks the half, so the slot must differ over the eight rows of each
//                  (parity class, row % 2): 2 (j % 4) + (row / 2) % 2 does;
//   32-byte rows:  row % 8 picks the eighth, so rows r and r + 8 / r + 24 of a class must
//                  differ: (row / 8) % 2 does.
// Row steps of a load item are multiples of 32, so a lane's swizzled slot is the same for
// every item.
template <int SPR>
__device__ __forceinline__ int slot_swizzle(int row) {
    if constexpr (SPR == 8) return (((row >> 2) & 3) << 1) | ((row >> 1) & 1);
    else if constexpr (SPR == 4) return (row >> 2) & 3;
    else return (row >> 3) & 1;
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

// Workgroup barrier for the stage ring.  Unlike __syncthreads() it carries no memory fence,
// so the LDS-DMA loads of later stages stay in flight across it; the stage it publishes was
// already waited for with an explicit vmcnt.  The "memory" clobber keeps the compiler from
// moving LDS accesses across it, the scheduling barriers keep register-only work (MFMAs) of one
// stage from drifting past the next stage's barrier.
__device__ __forceinline__ void stage_barrier() {
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_barrier" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
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

// Tile order of an M-grouped contiguous GEMM with a psum layout: the M-blocks of one expert's
// N-block take consecutive tile indices, so they run at the same time on one XCD and share the
// expert's weight tile in its L2 (the bands of swizzle_tile cut across experts).  Experts in
// order, each expert's N-blocks in order; the blocks past the last group's aligned end (zero
// tiles) come last.  Expert e's rows are [align(psum[e-1]), align(psum[e])); alignment is a
// multiple of BM.  Each wave scans 64 experts per round: a lane per expert, a prefix sum of their
// tile counts over the lanes.
__device__ __forceinline__ void expert_major_tile(const int* psum, int num_groups, int alignment, int t, int bm,
                                                  int nm, int nn, int& mb, int& nb) {
    const int lane = threadIdx.x & 63;
    int before = 0;   // tiles of the experts of earlier rounds
    for (int base = 0; base < num_groups; base += 64) {
        const int e = base + lane;
        int start = 0, end = 0;
        if (e < num_groups) {
            start = e == 0 ? 0 : align_up(psum[e - 1], alignment);
            end = align_up(psum[e], alignment);
        }
        const int blocks = max(0, end - start) / bm;
        const int tiles = blocks * nn;
        int incl = tiles;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const int v = __shfl_up(incl, off, 64);
            if (lane >= off) incl += v;
        }
        const uint64_t hit = __ballot(e < num_groups && t < before + incl);
        if (hit != 0) {
            const int src = __builtin_ctzll(hit);
            const int l = t - before - __shfl(incl - tiles, src, 64);
            const int bl = __shfl(blocks, src, 64);
            nb = l / bl;
            mb = __shfl(start, src, 64) / bm + l % bl;
            return;
        }
        before += __shfl(incl, 63, 64);
    }
    const int first = min(nm, align_up(psum[num_groups - 1], alignment) / bm);
    const int rest = max(1, nm - first);
    const int l = t - before;
    nb = min(nn - 1, l / rest);
    mb = min(nm - 1, first + l % rest);
}

// Segments of anchored tiles: with `runs` null, group e of a psum layout, rows
// [align(psum[e-1]), align(psum[e])), valid rows up to psum[e]; else run e of an m_indices layout
// (csrc/status.hip, m_indices_runs: runs[0] = count, then first row, group id and valid end per
// run), rows up to the next run's first row (the last: m_total), valid up to the run's valid end
// (rows of another id before it are zeroed by the epilogue).
struct Segment {
    int start, end, valid, group;
};
__device__ __forceinline__ int segment_count(const int* psum, int num_groups, const int* runs) {
    return runs != nullptr ? runs[0] : num_groups;
}
__device__ __forceinline__ Segment segment_at(const int* psum, int alignment, const int* runs, int count, int e,
                                              int m_total) {
    Segment sg;
    if (runs != nullptr) {
        sg.start = runs[1 + 3 * e];
        sg.end = e + 1 < count ? runs[4 + 3 * e] : m_total;
        sg.valid = runs[3 + 3 * e];
        sg.group = runs[2 + 3 * e];
    } else {
        sg.start = e == 0 ? 0 : align_up(psum[e - 1], alignment);
        sg.end = align_up(psum[e], alignment);
        sg.valid = psum[e];
        sg.group = e;
    }
    return sg;
}

// Number of anchored tiles of a launch (the tiles of every segment, then -- psum layouts -- the zero
// tiles of the rows past the last group): the grid is an upper bound, and only this many
// workgroups take a tile.
__device__ __forceinline__ int anchored_total(const int* psum, int num_groups, const int* runs, int alignment, int bm,
                                              int m_total, int nn) {
    const int lane = threadIdx.x & 63;
    const int count = segment_count(psum, num_groups, runs);
    int chunks = 0;
    for (int base = 0; base < count; base += 64) {
        const int e = base + lane;
        if (e < count) {
            const Segment sg = segment_at(psum, alignment, runs, count, e, m_total);
            chunks += ceil_div(max(0, sg.end - sg.start), bm);
        }
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) chunks += __shfl_xor(chunks, off, 64);
    if (runs == nullptr) chunks += ceil_div(max(0, m_total - align_up(psum[num_groups - 1], alignment)), bm);
    return chunks * nn;
}

// Anchored tiles of an M-grouped GEMM: each segment's rows are cut into chunks of BM rows starting
// at its first row, so a tile never mixes groups and a group of up to BM rows is one tile row
// (its weight tile streamed once, whatever the alignment).  Tiles run segment-major as in
// expert_major_tile; then (psum) chunks of the rows past the last group's aligned end (zero
// tiles).  Outputs: the group (-1: zero tile, -2: no tile), the tile's first row, N-block, the end
// of its rows (rows at or past it belong to another tile) and of its valid rows.
__device__ __forceinline__ void anchored_tile(const int* psum, int num_groups, const int* runs, int alignment, int t,
                                              int bm, int m_total, int nn, int& group, int& m0, int& nb, int& tile_end,
                                              int& valid_end) {
    const int lane = threadIdx.x & 63;
    const int count = segment_count(psum, num_groups, runs);
    int before = 0;
    for (int base = 0; base < count; base += 64) {
        const int e = base + lane;
        Segment sg = {0, 0, 0, -1};
        if (e < count) sg = segment_at(psum, alignment, runs, count, e, m_total);
        const int chunks = ceil_div(max(0, sg.end - sg.start), bm);
        const int tiles = chunks * nn;
        int incl = tiles;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const int v = __shfl_up(incl, off, 64);
            if (lane >= off) incl += v;
        }
        const uint64_t hit = __ballot(e < count && t < before + incl);
        if (hit != 0) {
            const int src = __builtin_ctzll(hit);
            const int l = t - before - __shfl(incl - tiles, src, 64);
            const int ch = __shfl(chunks, src, 64);
            group = __shfl(sg.group, src, 64);
            nb = l / ch;
            m0 = __shfl(sg.start, src, 64) + (l % ch) * bm;
            tile_end = min(m0 + bm, __shfl(sg.end, src, 64));
            valid_end = min(tile_end, __shfl(sg.valid, src, 64));
            if (valid_end <= m0 || group < 0 || group >= num_groups) group = -1;
            return;
        }
        before += __shfl(incl, 63, 64);
    }
    const int last = runs != nullptr ? m_total : align_up(psum[num_groups - 1], alignment);
    const int chunks = ceil_div(max(0, m_total - last), bm);
    const int l = t - before;
    if (chunks == 0 || l >= chunks * nn) {
        group = -2;
        return;
    }
    group = -1;
    nb = l / chunks;
    m0 = last + (l % chunks) * bm;
    tile_end = min(m0 + bm, m_total);
    valid_end = m0;
}

typedef float f32x16 __attribute__((ext_vector_type(16)));

// Old D values of a full 32-column block (accumulate), read ahead of its epilogue_block so that a
// wave issues the reads of several blocks before waiting for any (the lane's 16 values, in the
// accumulator's element order); zeros where epilogue_block reads D itself (ragged blocks).
template <int EPI>
__device__ __forceinline__ void load_old_block(const KParams& p, const uint8_t* d_base, int m, bool row_ok, int nblk,
                                               int N, int q, float (&old)[16]) {
    constexpr bool kF32 = EPI == kEpiF32;
    using OutT = typename Cond<kF32, float, uint16_t>::type;
    const OutT* drow = reinterpret_cast<const OutT*>(d_base) + (int64_t)m * p.ldd;
    const bool full = p.vec_store && nblk + 32 <= N;
#pragma unroll
    for (int i = 0; i < 16; ++i) old[i] = 0.f;
    if (full && row_ok) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            if constexpr (kF32) {
                const f32x4 o = *reinterpret_cast<const f32x4*>(drow + nblk + 8 * g + 4 * q);
#pragma unroll
                for (int i = 0; i < 4; ++i) old[4 * g + i] = o[i];
            } else {
                const i32x2 o = *reinterpret_cast<const i32x2*>(drow + nblk + 8 * g + 4 * q);
                old[4 * g + 0] = bf16_to_f32((uint16_t)(o[0] & 0xffff));
                old[4 * g + 1] = bf16_to_f32((uint16_t)((uint32_t)o[0] >> 16));
                old[4 * g + 2] = bf16_to_f32((uint16_t)(o[1] & 0xffff));
                old[4 * g + 3] = bf16_to_f32((uint16_t)((uint32_t)o[1] >> 16));
            }
        }
    }
}

// Epilogue of one 32x32 accumulator block: lane (r, q) holds output row m (the caller's
// row_ok / pad_row flags describe it) and columns nblk + 8 g + 4 q + {0..3} in elements
// 4 g + {0..3}; alpha, bias, accumulate, the D dtype (EPI) and stochastic rounding / FP8
// quantisation are applied here and the block is stored to D (d_base already offset by batch).
// old_pre: the block's old D values read ahead (load_old_block), or nullptr to read them here.
template <int EPI>
__device__ __forceinline__ void epilogue_block(const KParams& p, const f32x16& acc, uint8_t* d_base, int m,
                                               bool row_ok, bool pad_row, int nblk, int N, int batch, int q,
                                               const float* old_pre = nullptr) {
    const float alpha = p.alpha;
    constexpr bool kF32 = EPI == kEpiF32;
    constexpr bool kSR = EPI == kEpiBf16SR;
    constexpr bool kFp8 = EPI == kEpiFp8;
    using OutT = typename Cond<kF32, float, typename Cond<kFp8, uint8_t, uint16_t>::type>::type;
    OutT* drow = reinterpret_cast<OutT*>(d_base) + (int64_t)m * p.ldd;
    const OutT* bp = reinterpret_cast<const OutT*>(p.bias);
    const bool acc_old = p.accumulate, bias = p.has_bias, vec = p.vec_store;
    auto to_f = [](OutT x) -> float {
        if constexpr (kF32) return x; else if constexpr (kFp8) return 0.f; else return bf16_to_f32(x);
    };
    // the lane holds columns nblk + 8 g + 4 q + {0..3} in elements 4 g + {0..3}
    float v[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) v[i] = acc[i] * alpha;
    if constexpr (kFp8) {
        // Quantise the bf16-rounded outputs per 32 columns of a row: this lane holds 16 of
        // them, its partner lane (q ^ 1) the other 16.  The host guarantees n % 128 == 0, so
        // a block is either entirely inside the row or entirely past it.
        uint32_t amax = 0;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const uint16_t h = f32_to_bf16_rne(v[i]);
            v[i] = bf16_to_f32(h);
            amax = max(amax, (uint32_t)(h & 0x7fffu));
        }
        amax = max(amax, (uint32_t)__shfl_xor((int)amax, 32));
        const uint32_t sexp = ue8m0_of_bf16_amax(amax);
        const float inv = __builtin_bit_cast(float, (254u - sexp) << 23);   // 2^(127 - s)
        if (row_ok && nblk < N) {
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                int w = __builtin_amdgcn_cvt_pk_fp8_f32(v[4 * g] * inv, v[4 * g + 1] * inv, 0, false);
                w = __builtin_amdgcn_cvt_pk_fp8_f32(v[4 * g + 2] * inv, v[4 * g + 3] * inv, w, true);
                *reinterpret_cast<int*>(drow + nblk + 8 * g + 4 * q) = w;
            }
            if (q == 0) {
                const int64_t col = (int64_t)batch * N + nblk;
                p.sfd[((col >> 6) * p.sfd_ld + m) * 2 + ((col >> 5) & 1)] = (uint8_t)sexp;
            }
        }
    } else {
    const bool full = vec && nblk + 32 <= N;                   // wave-uniform
    if (full) {
        if (bias) {
#pragma unroll
            for (int g = 0; g < 4; ++g)
#pragma unroll
                for (int i = 0; i < 4; ++i) v[4 * g + i] += to_f(bp[nblk + 8 * g + 4 * q + i]);
        }
        if (acc_old && row_ok) {
            if (old_pre != nullptr) {
#pragma unroll
                for (int i = 0; i < 16; ++i) v[i] += old_pre[i];
            } else {
#pragma unroll
                for (int g = 0; g < 4; ++g)
#pragma unroll
                    for (int i = 0; i < 4; ++i) v[4 * g + i] += to_f(drow[nblk + 8 * g + 4 * q + i]);
            }
        }
        if constexpr (kF32) {
            if (row_ok) {
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    f32x4 o = {v[4 * g], v[4 * g + 1], v[4 * g + 2], v[4 * g + 3]};
                    if (pad_row) o = f32x4{0.f, 0.f, 0.f, 0.f};
                    *reinterpret_cast<f32x4*>(drow + nblk + 8 * g + 4 * q) = o;
                }
            }
        } else {
            // pk[g] = columns 8 g + 4 q + {0..3} as two bf16 pairs
            uint32_t pk[4][2];
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                if constexpr (kSR) {
                    uint16_t o[4];
                    sr_bf16_quartet(v + 4 * g, (uint32_t)(nblk + 8 * g + 4 * q) >> 2, o);
                    pk[g][0] = pad_row ? 0u : (uint32_t)o[0] | ((uint32_t)o[1] << 16);
                    pk[g][1] = pad_row ? 0u : (uint32_t)o[2] | ((uint32_t)o[3] << 16);
                } else {
                    pk[g][0] = pad_row ? 0u : pack_bf16x2(v[4 * g], v[4 * g + 1]);
                    pk[g][1] = pad_row ? 0u : pack_bf16x2(v[4 * g + 2], v[4 * g + 3]);
                }
            }
            // v_permlane32_swap regroups the wave halves: afterwards the lower half
            // (q = 0) holds columns 16..31 and the upper half (q = 1) columns 0..15 of
            // the block, i.e. 32 contiguous bytes per lane.
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const auto s02 = __builtin_amdgcn_permlane32_swap(pk[2][h], pk[0][h], false, false);
                const auto s13 = __builtin_amdgcn_permlane32_swap(pk[3][h], pk[1][h], false, false);
                pk[2][h] = s02[0]; pk[0][h] = s02[1];
                pk[3][h] = s13[0]; pk[1][h] = s13[1];
            }
            if (row_ok) {
                // q = 0: pk2 = 16..19, pk0 = 20..23, pk3 = 24..27, pk1 = 28..31
                // q = 1: pk2 = 0..3,   pk0 = 4..7,   pk3 = 8..11,  pk1 = 12..15
                uint16_t* dp = drow + nblk + (q ? 0 : 16);
                *reinterpret_cast<i32x4*>(dp) = i32x4{(int)pk[2][0], (int)pk[2][1], (int)pk[0][0], (int)pk[0][1]};
                *reinterpret_cast<i32x4*>(dp + 8) = i32x4{(int)pk[3][0], (int)pk[3][1], (int)pk[1][0], (int)pk[1][1]};
            }
        }
    } else if (row_ok && kSR) {
        // ragged / unaligned block, stochastic rounding: columns past the row hash as zeros
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int n = nblk + 8 * g + 4 * q;
            float x[4];
            uint16_t o[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) x[i] = n + i < N ? v[4 * g + i] : 0.f;
            sr_bf16_quartet(x, (uint32_t)n >> 2, o);
#pragma unroll
            for (int i = 0; i < 4; ++i)
                if (n + i < N) drow[n + i] = pad_row ? (uint16_t)0 : o[i];
        }
    } else if (row_ok) {
        // ragged / unaligned block: element stores with bounds
#pragma unroll
        for (int g = 0; g < 4; ++g)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int n = nblk + 8 * g + 4 * q + i;
                if (n < N) {
                    float x = v[4 * g + i];
                    if (bias) x += to_f(bp[n]);
                    if (acc_old) x += to_f(drow[n]);
                    if constexpr (kF32) drow[n] = pad_row ? 0.f : x;
                    else drow[n] = pad_row ? (uint16_t)0 : f32_to_bf16_rne(x);
                }
            }
    }
    }   // !kFp8
}

// The kernel body.  OCC = workgroups per CU the kernel is compiled for (its waves per SIMD bound
// its registers).  CT / CS / CM / CN / CK fix the GEMM type, the K split and M / N / K at compile
// time (-1 / 0 = read from the arguments): the ahead-of-time menu reads everything from the
// arguments, the JIT compiles one body per problem (csrc/jit.hip).
template <int BM, int BN, int WGM, int NW, int LW, int NSTAGE, int KM, int OCC, int KIND, int EPI, int CT = -1,
          int CS = 0, int CM = 0, int CN = 0, int CK = 0, bool AMN = false, bool BMN = false, int NSB_ = 0>
__device__ __forceinline__ void gemm_body(const KParams& p, const int vb, const int known_total = -1) {
    constexpr bool kAFp4 = KIND == kFP4FP4;
    constexpr bool kBFp4 = KIND == kFP8FP4 || KIND == kFP4FP4;
    constexpr bool kBf16 = KIND == kBF16;
    constexpr int kFmtA = kAFp4 ? kFmtE2M1 : kFmtE4M3;
    constexpr int kFmtB = kBFp4 ? kFmtE2M1 : kFmtE4M3;
    // A stage holds KM sub-steps of one MFMA K-step each (64 fp8 / fp4 or 32 bf16 elements).
    // KM = 2 makes fp8 / bf16 rows 128 bytes per stage: every global load then fetches whole
    // 128-byte lines (measured 1.5x the LDS-fill rate of 64-byte row pieces).
    static_assert(KM == 1 || KM == 2, "sub-steps per stage");
    constexpr int KS = (kBf16 ? 32 : 64) * KM;           // K elements per stage
    constexpr int RBA = (kAFp4 ? 32 : 64) * KM;          // bytes of one row per stage
    constexpr int RBB = (kBFp4 ? 32 : 64) * KM;
    constexpr int SPRA = RBA / 16, SPRB = RBB / 16;
    // With three or more ring slots the next stage has landed while this one computes, so its
    // first fragments are read ahead across the stage barrier.  A two-slot ring (128-K stages of
    // the largest tiles, KM = 2) syncs late instead: once a stage's last fragments are in
    // registers, before its last MFMA group, the waves wait for the next stage, meet at the
    // barrier, refill the slot just drained and read the next stage's first fragments while
    // that group's MFMAs run -- so no stage starts on an empty MFMA pipe.
    constexpr bool kCross = NSTAGE >= 3;
    constexpr bool kLate = NSTAGE == 2;
    // Late-sync rings issue the next stage's loads spread over the first sub-step's MFMA groups
    // (kSpread) or all at the sync point.
    constexpr bool kSpread = false;
    static_assert(!kLate || KM == 2, "two-slot rings need 128-byte stages");
    constexpr int NT = NW * 64;                          // threads per workgroup
    // The last LW waves issue every global->LDS load; with LW < NW the other waves only read
    // LDS and run MFMAs, so a stall in the load-issue path never blocks a whole SIMD.
    constexpr int LT = LW * 64, FW = NW - LW;            // loader threads, first loader wave
    static_assert(LW == NW || (NW == 8 && LW == 4), "loader waves");
    constexpr int WGN = NW / WGM;
    constexpr int WM = BM / WGM;                         // wave tile rows
    constexpr int WN = (BN / WGN + 31) / 32 * 32;        // wave tile columns (32-column blocks)
    constexpr int TM = WM / 32, TN = WN / 32;            // 32x32 MFMA blocks per wave
    // Ragged wave tiling: the last wave column holds TN_LAST < TN blocks (256x224 = 4 + 3
    // blocks of 32 columns).  Those waves are exactly the loader waves (waves 4..7 with 4 waves
    // along M), and each SIMD runs one wave of each column, so every SIMD still issues the
    // same number of MFMAs per stage while the loader waves carry fewer.
    constexpr int TN_LAST = (BN - (WGN - 1) * WN) / 32;
    constexpr bool kRagged = TN_LAST != TN;
    static_assert((NW == 4 || NW == 8) && WGM * WGN == NW && TM >= 1 && TN >= 1 && TM * 32 == WM &&
                      TN_LAST >= 1 && (WGN - 1) * WN + TN_LAST * 32 == BN, "wave tiling");
    static_assert(!kRagged || (NW == 8 && LW == 4 && WGM == 4 && WGN == 2), "ragged tiling needs the loader waves as its last column");
    // MN-major operands (AMN / BMN: A [K][M] / B [K][N], MN contiguous; e4m3 or bf16, 128-byte stages):
    // a stage holds the tile's K rows (128 e4m3 / 64 bf16) of up to 256 MN elements each, in LDS rows
    // of 256 elements whose 16-byte pieces are XOR-swizzled (e4m3: by 2 (k % 8), bf16: by 4 (k % 4));
    // fragments are read with ds_read_b64_tr_b8 / _b16, which hand each lane consecutive K of one MN
    // row, so the MFMA operands equal the K-major path's.
    static_assert((!AMN && !BMN) || ((KIND == kFP8FP8 || KIND == kBF16) && KM == 2 && NSTAGE == 2 &&
                                     (!AMN || BM <= 256) && (!BMN || BN <= 256)),
                  "MN-major operands: e4m3 or bf16, 128-byte stages, at most 256 MN rows per operand tile");
    constexpr int MN_E = kBf16 ? 2 : 1;                    // bytes per element
    constexpr int MN_PITCH = 256 * MN_E, MN_KROWS = KS;   // an MN-major stage: KS K rows x 256 elements
    constexpr int MN_PPR = MN_PITCH / 16;                 // 16-byte pieces per LDS row
    // piece swizzle of MN-major LDS row k: the K rows one transposing read touches (8 for e4m3, 4 for
    // bf16) land on distinct bank groups, and so do the two 16-lane groups served together
    auto mn_swizzle = [](int k) -> int { return kBf16 ? (k & 3) << 2 : (k & 7) << 1; };
    constexpr int A_BYTES = AMN ? MN_KROWS * MN_PITCH : BM * RBA, B_BYTES = BMN ? MN_KROWS * MN_PITCH : BN * RBB;
    constexpr int SCA = kBf16 ? 0 : (BM * 2 + 255) / 256 * 256;   // one packed int16 per row and sub-step
    constexpr int SCB = kBf16 ? 0 : (BN * 2 + 255) / 256 * 256;
    constexpr int SCU = SCA + SCB;                                 // scale bytes of one sub-step
    constexpr int NSCA = kBf16 ? 0 : (BM + 127) / 128, NSCB = kBf16 ? 0 : (BN + 127) / 128;
    // 256 idle bytes per stage that take the dead SF loads of waves without an SF row to fetch
    constexpr int SPARE = (!kBf16 && NSCA + NSCB < LW) ? 256 : 0;
    // Split ring (NSB = 3 B slots beside a two-slot late-sync ring of A + SF): B rows get a ring of
    // their own, one slot deeper, and each late sync issues A / SF of stage c + 2 and B of stage
    // c + 3.  A CU's load rate follows the bytes it keeps in flight (measured on MI355X), and the
    // deeper B ring holds ~1.5x the bytes of one stage in flight within the 160 KB of LDS.
    // NSB_ requests it; the kernel takes it where it fits the LDS (otherwise one shared ring).
    constexpr int STAGE = A_BYTES + B_BYTES + KM * SCU + SPARE;     // unified ring slot
    constexpr bool kSplitRing = NSB_ == 3 && NSTAGE == 2 && KM == 2 && !AMN && !BMN &&
                                (NSTAGE * (STAGE - B_BYTES) + NSB_ * B_BYTES) * OCC <= 160 * 1024;
    constexpr int NSB = kSplitRing ? NSB_ : NSTAGE;
    constexpr int STAGE_A = kSplitRing ? A_BYTES + KM * SCU + SPARE : STAGE;   // slot of A (+ SF)
    constexpr int SC_OFF = kSplitRing ? A_BYTES : A_BYTES + B_BYTES;          // SF area within it
    constexpr int RING_A = NSTAGE * STAGE_A;
    constexpr int LDS_BYTES = kSplitRing ? RING_A + NSB * B_BYTES : NSTAGE * STAGE;
    static_assert(NSTAGE >= 2 && LDS_BYTES * OCC <= 160 * 1024, "LDS budget");
    __shared__ __attribute__((aligned(1024))) uint8_t smem[LDS_BYTES];
    auto a_slot = [&](int s) -> uint8_t* { return smem + s * STAGE_A; };
    auto b_slot = [&](int sb) -> uint8_t* { return kSplitRing ? smem + RING_A + sb * B_BYTES : smem + sb * STAGE + A_BYTES; };

    int tid = threadIdx.x;
    // In the persistent walk (known_total >= 0) the thread index is made opaque on every tile, so the
    // per-lane load and fragment offsets derived from it are recomputed per tile instead of being hoisted
    // out of the walk and held live across the main loop (they spilled the 384-row walk, ~290 bytes per
    // lane).  A one-tile launch passes -1 and keeps its code as it was.
    if (known_total >= 0) asm volatile("" : "+v"(tid));
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lwave = wave - FW, ltid = tid - FW * 64;   // loader wave / thread index
    const bool is_loader = lwave >= 0;
    const int wm = wave % WGM, wn = wave / WGM;
    const int r = lane & 31, q = lane >> 5;

    // ------------------------------------------------------------------ tile selection
    const int gemm_type = CT >= 0 ? CT : p.gemm_type;
    const int split_k = CS > 0 ? CS : p.split_k;
    const int nm = CM > 0 ? ceil_div(CM, BM) : p.num_m_blocks, nn = CN > 0 ? ceil_div(CN, BN) : p.num_n_blocks;
    int t, split = 0;
    if (split_k > 1) {
        // Split-K launch: grid = 8 * ceil(tiles / 8) * split_k, and workgroup b serves tile
        // (b / 8 / split_k) * 8 + b % 8, split (b / 8) % split_k, so all splits of a tile share
        // b % 8 -- the XCD (and L2) the dispatcher places them on.
        const int b = vb, r = b >> 3;
        t = (r / split_k) * 8 + (b & 7);
        split = r % split_k;
        if (p.split_spread) {
            // (test knob: consecutive workgroups -- different XCDs -- take the splits of a tile)
            t = b / split_k;
            split = b % split_k;
        }
        if (t >= p.num_tiles) return;
    } else if (gemm_type == kKGrouped) {
        // K-grouped: each group's tiles are spread over the XCDs on their own, so at any time all
        // XCDs work on one group and its A / B K-slices (Kg x (M + N) bytes) are streamed once,
        // instead of every XCD pair streaming another group's and the groups together overflowing
        // the last-level cache.  (groups in order; a group's tiles are consecutive workgroups)
        const int per_group = nm * nn;
        const int g = vb / per_group;
        t = g * per_group + xcd_remap(vb - g * per_group, per_group);
    } else {
        t = xcd_remap(vb, p.vgrid);
    }
    const int tile_id = t;
    int batch = 0;
    if (gemm_type == kBatched || gemm_type == kMasked || gemm_type == kKGrouped) {
        batch = t / (nm * nn);
        t -= batch * nm * nn;
    }
    const int M = CM > 0 ? CM : p.m, N = CN > 0 ? CN : p.n;
    int mb = 0, nb = 0, m0, anchor_group = -1, tile_end = M, anchor_valid = M;
    const bool anchored = (gemm_type == kMGroupedPsum || gemm_type == kMGroupedIdx) && p.anchored && p.num_groups > 0;
    if (anchored) {
        const int* runs = gemm_type == kMGroupedIdx ? p.runs : nullptr;
        // the launch's real tiles spread over the XCDs as xcd_remap spreads a full grid
        const int total = known_total >= 0 ? known_total
            : __builtin_amdgcn_readfirstlane(anchored_total(p.layout, p.num_groups, runs, p.alignment, BM, M, nn));
        if (vb >= total) return;
        t = xcd_remap(vb, total);
        anchored_tile(p.layout, p.num_groups, runs, p.alignment, t, BM, M, nn, anchor_group, m0, nb, tile_end,
                      anchor_valid);
        anchor_group = __builtin_amdgcn_readfirstlane(anchor_group);
        if (anchor_group == -2) return;   // past the last tile of this launch
        m0 = __builtin_amdgcn_readfirstlane(m0);
        nb = __builtin_amdgcn_readfirstlane(nb);
        tile_end = __builtin_amdgcn_readfirstlane(tile_end);
        anchor_valid = __builtin_amdgcn_readfirstlane(anchor_valid);
    } else {
        if (gemm_type == kMGroupedPsum && p.num_groups > 0)
            expert_major_tile(p.layout, p.num_groups, p.alignment, t, BM, nm, nn, mb, nb);
        else
            swizzle_tile(t, nm, nn, p.group_m, mb, nb);
        mb = __builtin_amdgcn_readfirstlane(mb);
        nb = __builtin_amdgcn_readfirstlane(nb);
        m0 = mb * BM;
    }
    const int n0 = nb * BN;

    const uint8_t* a_base = p.a;
    const uint8_t* b_base = p.b;
    const uint16_t* sfa = p.sfa;
    const uint16_t* sfb = p.sfb;
    uint8_t* d_base = p.d;
    const int out_esize = p.out_esize;
    int group = 0;          // B operand group
    int valid_end = M;      // rows >= valid_end are padding (psum) / not written (masked)
    bool zero_tile = false;
    int k_len = CK > 0 ? CK : p.k;   // K extent of this tile's contraction

    if (gemm_type == kKGrouped) {
        // K-grouped: group g contracts K rows [align(psum[g-1]), psum[g]) of A and B into D[g].
        const int ks = batch == 0 ? 0 : align_up(p.layout[batch - 1], p.alignment);
        k_len = __builtin_amdgcn_readfirstlane(max(0, p.layout[batch] - ks));
        const int kso = __builtin_amdgcn_readfirstlane(ks);
        a_base += AMN ? (int64_t)kso * p.lda : (int64_t)kso * (kAFp4 ? 1 : (kBf16 ? 4 : 2)) / 2;
        b_base += BMN ? (int64_t)kso * p.ldb : (int64_t)kso * (kBFp4 ? 1 : (kBf16 ? 4 : 2)) / 2;
        // (p.lda / p.ldb are in bytes: an MN-major K row is lda bytes)
        if (!kBf16) {
            sfa += (int64_t)(kso / 64) * p.sfa_ld;
            sfb += (int64_t)(kso / 64) * p.sfb_ld;
        }
        d_base += (int64_t)batch * p.bsd * out_esize;
    }

    if (gemm_type == kBatched || gemm_type == kMasked) {
        group = batch;
        a_base += (int64_t)batch * p.bsa;
        d_base += (int64_t)batch * p.bsd * out_esize;
        if (!kBf16) sfa += (int64_t)batch * p.sfa_bs;
        if (gemm_type == kMasked) {
            valid_end = min(M, p.layout[batch]);
            if (m0 >= valid_end) return;   // whole tile beyond masked_m: nothing to write
        }
    } else if (anchored) {
        group = anchor_group;
        valid_end = anchor_valid;
        if (group < 0) zero_tile = true;
    } else if (gemm_type == kMGroupedPsum) {
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
    } else if (gemm_type == kMGroupedIdx) {
        group = __builtin_amdgcn_readfirstlane(p.layout[m0]);
        // (padding rows, and ids past the last group -- which the m_indices check reports --
        // read no B)
        if (group < 0 || group >= p.num_groups) zero_tile = true;
    }
    group = __builtin_amdgcn_readfirstlane(group);
    valid_end = __builtin_amdgcn_readfirstlane(valid_end);

    if (zero_tile) {
        // Padding-only tile of an M-grouped layout: its D rows are exact zeros (16-byte stores when
        // the rows allow them).
        const int rows = min(BM, tile_end - m0), cols = min(BN, N - n0);
        const int row_bytes = cols * out_esize;
        uint8_t* d0 = d_base + ((int64_t)m0 * p.ldd + n0) * out_esize;
        const int64_t ld_bytes = p.ldd * out_esize;
        if (row_bytes % 16 == 0 && ld_bytes % 16 == 0 && (reinterpret_cast<uint64_t>(d0) & 15) == 0) {
            const int per_row = row_bytes / 16;
            for (int e = tid; e < rows * per_row; e += NT)
                *reinterpret_cast<i32x4*>(d0 + (int64_t)(e / per_row) * ld_bytes + (e % per_row) * 16) = i32x4{0, 0, 0, 0};
        } else {
            for (int e = tid; e < rows * cols; e += NT) {
                const int rr = e / cols, cc = e % cols;
                const int64_t off = (int64_t)(m0 + rr) * p.ldd + n0 + cc;
                if (out_esize == 4) reinterpret_cast<float*>(d_base)[off] = 0.f;
                else reinterpret_cast<uint16_t*>(d_base)[off] = 0;
            }
        }
        return;
    }
    if (gemm_type != kNormal && gemm_type != kKGrouped) {
        b_base += (int64_t)group * p.bsb;
        if (!kBf16) sfb += (int64_t)group * p.sfb_bs;
    }

    // (an anchored tile loads only its group's valid rows: the rest of the tile reads zeros)
    const int rows_a = anchored ? min(BM, valid_end - m0) : min(BM, M - m0);
    const int rows_b = min(BN, N - n0);
    const int64_t lda = p.lda, ldb = p.ldb;
    // (MN-major: the tile's first column is the base and the K rows of the contraction bound the
    // range, so K rows past the end read zeros)
    const __amdgpu_buffer_rsrc_t rs_a = AMN ? make_rsrc(a_base + m0 * MN_E, (int64_t)k_len * lda - m0 * MN_E)
                                            : make_rsrc(a_base + (int64_t)m0 * lda, (int64_t)rows_a * lda);
    const __amdgpu_buffer_rsrc_t rs_b = BMN ? make_rsrc(b_base + n0 * MN_E, (int64_t)k_len * ldb - n0 * MN_E)
                                            : make_rsrc(b_base + (int64_t)n0 * ldb, (int64_t)rows_b * ldb);
    // (bytes of one K row: storage bytes per two K elements x K / 2)
    const int kbytes_a = gemm_type == kKGrouped || CK > 0 ? k_len * (kAFp4 ? 1 : (kBf16 ? 4 : 2)) / 2 : p.kbytes_a;
    const int kbytes_b = gemm_type == kKGrouped || CK > 0 ? k_len * (kBFp4 ? 1 : (kBf16 ? 4 : 2)) / 2 : p.kbytes_b;
    // With KM = 1 the ring walks an even number of virtual stages so the main loop is a pair of
    // iterations with static register sets; an odd stage count gets one leading dead stage
    // (all-zero operands and scales, so it adds nothing to the accumulators).  With KM = 2 the
    // two sub-steps of every stage own the two register sets.
    // K stages of this workgroup: [c0, c0 + num_stages) of the whole K loop.
    const int c0 = split * p.split_stages;
    const int num_stages = split_k > 1 ? min(p.split_stages, ceil_div(k_len, KS) - c0) : ceil_div(k_len, KS);
    const int shift = KM == 1 ? (num_stages & 1) : 0;
    const int num_virtual = num_stages + shift;
    const int nk64 = ceil_div(k_len, 64);

    // ------------------------------------------------------------------ loads
    // Operand rows: each wave-level buffer_load_dwordx4 ... lds fills 1 KB (64 lanes x 16 B)
    // of a stage; lane slots map to swizzled (row, 16-byte K piece) positions.  The stage's K
    // offset rides in the scalar soffset, so the per-lane voffset is stage-invariant.
    constexpr int SLA = AMN ? MN_KROWS * MN_PPR : BM * SPRA, SLB = BMN ? MN_KROWS * MN_PPR : BN * SPRB;   // 16-byte slots per stage
    constexpr int NLA = (SLA + LT - 1) / LT, NLB = (SLB + LT - 1) / LT;  // per-thread loads
    // Packed SF rows: one buffer_load_dword ... lds per 128 rows of the tile and sub-step,
    // issued by waves 0 .. NSCA-1 (A) and NSCA .. NSCA+NSCB-1 (B).
    static_assert(NSCA + NSCB <= LW, "scale loads per stage");
    constexpr int NL = NLA + NLB + (kBf16 ? 0 : KM);
    // Loads that every wave issues per stage (the waits below count the smallest number).
    constexpr int kMinLoadsPerStage = (SLA / LT) + (SLB / LT) + (kBf16 ? 0 : KM);

    // Per-lane byte offset of the thread's first 16-byte slot of the A / B stage and the K piece
    // it covers; load item `it` adds it * LT / SPR rows through the scalar offset.
    int lk_a, lk_b;
    uint32_t vbase_a, vbase_b;
    {
        const int row_a = ltid / SPRA, row_b = ltid / SPRB;
        lk_a = ((ltid % SPRA) ^ slot_swizzle<SPRA>(row_a)) * 16;
        lk_b = ((ltid % SPRB) ^ slot_swizzle<SPRB>(row_b)) * 16;
        vbase_a = row_a < rows_a ? (uint32_t)(row_a * lda + lk_a) : kOOBOffset;
        vbase_b = row_b < rows_b ? (uint32_t)(row_b * ldb + lk_b) : kOOBOffset;
        // MN-major: LDS slot ltid = K row ltid / MN_PPR, piece ltid % MN_PPR of the swizzled row,
        // which holds MN bytes [16 pp, 16 pp + 16) with pp = piece ^ mn_swizzle(k); pieces past the
        // tile's MN extent read zeros
        const int kr = ltid / MN_PPR, pp = (ltid % MN_PPR) ^ mn_swizzle(kr);
        if constexpr (AMN) vbase_a = pp * 16 < rows_a * MN_E ? (uint32_t)(kr * lda + pp * 16) : kOOBOffset;
        if constexpr (BMN) vbase_b = pp * 16 < rows_b * MN_E ? (uint32_t)(kr * ldb + pp * 16) : kOOBOffset;
    }
    const int vstep_a = __builtin_amdgcn_readfirstlane((int)(AMN ? (LT / MN_PPR) * lda : (LT / SPRA) * lda));
    const int vstep_b = __builtin_amdgcn_readfirstlane((int)(BMN ? (LT / MN_PPR) * ldb : (LT / SPRB) * ldb));
    // Per-wave packed-SF load of a stage: loader wave w < NSCA fetches A rows [128 w, 128 w + 128),
    // loader waves NSCA .. NSCA+NSCB-1 the B rows; the other waves issue a dead (out-of-range) load
    // into an idle word so that every wave runs the same branch-free instruction stream.
    __amdgpu_buffer_rsrc_t rs_sc;
    uint32_t sc_voff = kOOBOffset;
    int sc_step = 0, sc_lds = 0;
    bool sc_live = false;
    if constexpr (!kBf16) {
        const bool is_a = lwave < NSCA;
        const int w = is_a ? lwave : lwave - NSCA;
        sc_live = lwave >= 0 && lwave < NSCA + NSCB;
        rs_sc = is_a ? make_rsrc(sfa + m0, ((int64_t)nk64 * p.sfa_ld - m0) * 2)
                     : make_rsrc(sfb + n0, ((int64_t)nk64 * p.sfb_ld - n0) * 2);
        const int row = w * 128 + 2 * lane;
        sc_voff = (sc_live && row < (is_a ? rows_a : rows_b)) ? (uint32_t)(row * 2) : kOOBOffset;
        sc_step = __builtin_amdgcn_readfirstlane((int)((is_a ? p.sfa_ld : p.sfb_ld) * 2));
        sc_lds = __builtin_amdgcn_readfirstlane(sc_live ? SC_OFF + (is_a ? 0 : SCA) + w * 256 : SC_OFF + KM * SCU);
    }
    constexpr int kDeadOffset = 0x40000000;   // scalar offset that moves every lane out of range

    // Load item IDX of stage c into ring slot s.  `live == false` turns it into an
    // out-of-range load (zeros into an idle slot, no memory traffic) so that every wave keeps
    // the same instruction stream and the code stays branch-free for the scheduler.
    // (split ring: s is the B slot for B items)
    auto issue_item = [&](auto idx_tag, int c, int s, bool live) {
        constexpr int IDX = decltype(idx_tag)::value;
        uint8_t* sbase = a_slot(s);
        if constexpr (IDX < NLA + NLB) {
            constexpr bool kIsA = IDX < NLA;
            constexpr int it = kIsA ? IDX : IDX - NLA;
            constexpr int SL = kIsA ? SLA : SLB;
            constexpr int RB = kIsA ? RBA : RBB;
            if (SL % LT != 0 && it * LT + lwave * 64 >= SL) return;
            constexpr bool kMN = kIsA ? AMN : BMN;
            const int kb = kMN ? c * MN_KROWS * (int)(kIsA ? lda : ldb) : c * RB;
            const int krem = (kIsA ? kbytes_a : kbytes_b) - c * RB;
            // Rows past a ragged tile's edge fall outside the tile's buffer range and read zeros.
            // The item's row step rides in the scalar offset with the stage's K offset.  (MN-major:
            // K rows past the end fall outside the range instead.)
            const uint32_t voff = kMN || (kIsA ? lk_a : lk_b) < krem ? (kIsA ? vbase_a : vbase_b) : kOOBOffset;
            const int soff = kb + it * (kIsA ? vstep_a : vstep_b);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                kIsA ? rs_a : rs_b, (lds_void*)((kIsA ? sbase : b_slot(s)) + (it * LT + lwave * 64) * 16), 16,
                voff, __builtin_amdgcn_readfirstlane(live ? soff : kDeadOffset), 0, 0);
        } else if constexpr (!kBf16) {
            // packed-SF row of sub-step u of stage c (its k64 index is c * KM + u); a dead load
            // lands in the spare word, whatever u
            constexpr int u = IDX - NLA - NLB;
            const bool on = live & sc_live;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rs_sc, (lds_void*)(sbase + sc_lds + (sc_live ? u * SCU : 0)), 4,
                                                     sc_voff,
                                                     __builtin_amdgcn_readfirstlane(on ? (c * KM + u) * sc_step : kDeadOffset),
                                                     0, 0);
        }
    };
    auto issue_stage = [&](int c, int s, bool live) {
        static_for<NL>([&](auto i) { issue_item(i, c, s, live); });
    };
    // split ring: A rows and SF of stage c into A slot s, then B rows of stage cb into B slot sb
    // (issue order A, SF, B: a wait that leaves the last B items in flight covers A and SF)
    auto issue_split = [&](int c, int s, bool live, int cb, int sb, bool live_b) {
        static_for<NLA>([&](auto i) { issue_item(i, c, s, live); });
        static_for<NL - NLA - NLB>([&](auto i) { issue_item(Int<NLA + NLB + decltype(i)::value>{}, c, s, live); });
        static_for<NLB>([&](auto i) { issue_item(Int<NLA + decltype(i)::value>{}, cb, sb, live_b); });
    };
    constexpr int kMinLoadsB = SLB / LT;   // B items every loader wave issues per stage

    // ------------------------------------------------------------------ fragments
    auto frag_addr = [&](int R, int slot, auto spr_tag) -> int {
        constexpr int SPR = decltype(spr_tag)::value;
        return R * (SPR * 16) + ((slot ^ slot_swizzle<SPR>(R)) << 4);
    };
    // Sub-step u of row R: 32 bytes (fp8: K [16q,+16) and [32+16q,+16) of the sub-step; bf16:
    // its k-steps 0 and 1) or 16 bytes (fp4).  A sub-step spans 64 row bytes (32 for fp4).
    auto load_frag = [&](const uint8_t* base, int R, auto spr_tag, auto u_tag) -> i32x8 {
        constexpr int SPR = decltype(spr_tag)::value;
        constexpr int u = decltype(u_tag)::value;
        constexpr int P = SPR / KM;                      // 16-byte slots per sub-step
        const i32x4 lo = *reinterpret_cast<const i32x4*>(base + frag_addr(R, u * P + q, spr_tag));
        if constexpr (P == 4) {
            const i32x4 hi = *reinterpret_cast<const i32x4*>(base + frag_addr(R, u * P + 2 + q, spr_tag));
            return i32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        } else {
            return i32x8{lo[0], lo[1], lo[2], lo[3], 0, 0, 0, 0};
        }
    };
    // MN-major operand block starting at MN row R0 (its lane (r, q) = row R0 + r): four transposing
    // reads.  e4m3 (ds_read_b64_tr_b8):  In each 16-lane group (lanes 16 g + i, g = 2 q + h) lane s supplies
    // the 8-byte chunk of K row kb + s / 2 at MN bytes R0 + 16 h + 8 (s % 2); the read hands lane i
    // byte i % 8 of chunk 2 j + i / 8 as its byte j, i.e. K kb .. kb + 7 of MN row R0 + 16 h + i.
    // The four reads cover K [16 q, +8), [16 q + 8, +8), [32 + 16 q, +8), [40 + 16 q, +8) of the
    // sub-step: the K-major fragment's bytes in order.
    auto load_frag_mn = [&](const uint8_t* base, int R0, auto u_tag) -> i32x8 {
        constexpr int u = decltype(u_tag)::value;
        const int s16 = lane & 15, h = (lane >> 4) & 1;
        typedef int v2i __attribute__((ext_vector_type(2)));
        if constexpr (!kBf16) {
            const int pp = ((R0 + 16 * h) >> 4) ^ mn_swizzle(s16 >> 1);
            const uint8_t* b0 = base + (u * 64 + 16 * q + (s16 >> 1)) * MN_PITCH + (pp << 4) + (s16 & 1) * 8;
            typedef __attribute__((address_space(3))) v2i lds_v2i;
            const v2i e0 = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i*)(b0));
            const v2i e1 = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i*)(b0 + 8 * MN_PITCH));
            const v2i e2 = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i*)(b0 + 32 * MN_PITCH));
            const v2i e3 = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i*)(b0 + 40 * MN_PITCH));
            return i32x8{e0[0], e0[1], e1[0], e1[1], e2[0], e2[1], e3[0], e3[1]};
        } else {
            // ds_read_b64_tr_b16 (probed on gfx950): in each 16-lane group lane i receives element
            // i % 4 of the 4-element chunk addressed by source lane 4 j + i / 4 as its element j.  With
            // lane s addressing K row kb + s / 4 at MN elements R0 + 16 h + 4 (s % 4), lane i receives
            // K kb .. kb + 3 of MN row R0 + 16 h + i; four reads cover K [8 q, +8) and [16 + 8 q, +8) of
            // the sub-step's 32 K (the two 32x32x16 steps' operands).
            const int col = R0 + 16 * h + 4 * (s16 & 3);
            const int pp = (col >> 3) ^ mn_swizzle(s16 >> 2);
            const uint8_t* b0 = base + (u * 32 + 8 * q + (s16 >> 2)) * MN_PITCH + (pp << 4) + ((col >> 2) & 1) * 8;
            typedef short v4s __attribute__((ext_vector_type(4)));
            typedef __attribute__((address_space(3))) v4s lds_v4s;
            const v2i e0 = __builtin_bit_cast(v2i, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)(b0)));
            const v2i e1 = __builtin_bit_cast(v2i, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)(b0 + 4 * MN_PITCH)));
            const v2i e2 = __builtin_bit_cast(v2i, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)(b0 + 16 * MN_PITCH)));
            const v2i e3 = __builtin_bit_cast(v2i, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)(b0 + 20 * MN_PITCH)));
            return i32x8{e0[0], e0[1], e1[0], e1[1], e2[0], e2[1], e3[0], e3[1]};
        }
    };
    // UE8M0 byte of K-block q of row R (one packed int16 per row in the sub-step's scale area,
    // K-block 0 in the low byte): a byte read, consumed by the MFMA as it is.
    auto load_scale = [&](const uint8_t* sc, int R) -> int { return sc[R * 2 + q]; };

    f32x16 acc[TN][TM];
#pragma unroll
    for (int i = 0; i < TN; ++i)
#pragma unroll
        for (int j = 0; j < TM; ++j) acc[i][j] = f32x16{};

    // Register sets `buf` = 0 / 1 alternate between sub-steps (KM = 1: between stages): A-side
    // fragments and scales of the whole wave tile plus the first B-side block, all read one
    // sub-step ahead.
    i32x8 fa[2][TM];
    int sa[2][TM];
    i32x8 fb0[2];
    int sb0[2];
    auto load_ahead = [&](int s, int sb, auto part_tag, auto u_tag) {
        constexpr int part = decltype(part_tag)::value;   // TM: the B block, else A block `part`
        constexpr int u = decltype(u_tag)::value;
        const uint8_t* st = a_slot(s);
        const uint8_t* sc = st + SC_OFF + u * SCU;
        if constexpr (part < TM) {
            const int R = wm * WM + part * 32 + r;
            if constexpr (AMN) return Pair<i32x8, int>{load_frag_mn(st, R - r, u_tag), kBf16 ? 0 : load_scale(sc, R)};
            else return Pair<i32x8, int>{load_frag(st, R, Int<SPRA>{}, u_tag), kBf16 ? 0 : load_scale(sc, R)};
        } else {
            const int R = wn * WN + r;
            if constexpr (BMN) return Pair<i32x8, int>{load_frag_mn(b_slot(sb), R - r, u_tag), kBf16 ? 0 : load_scale(sc + SCA, R)};
            else return Pair<i32x8, int>{load_frag(b_slot(sb), R, Int<SPRB>{}, u_tag),
                                         kBf16 ? 0 : load_scale(sc + SCA, R)};
        }
    };
    auto prefetch = [&](int s, int sb, auto buf_tag, auto part_tag, auto u_tag) {
        constexpr int buf = decltype(buf_tag)::value;
        constexpr int part = decltype(part_tag)::value;
        const auto v = load_ahead(s, sb, part_tag, u_tag);
        if constexpr (part < TM) { fa[buf][part] = v.first; sa[buf][part] = v.second; }
        else { fb0[buf] = v.first; sb0[buf] = v.second; }
    };

    // Sub-step u of the stage in ring slot s with the registers of set `buf`.  Reads the ahead
    // registers of the next sub-step (u + 1 of this slot, or sub-step 0 of slot sn when the ring
    // crosses stages) into the other set, and -- in sub-step 0 -- issues the loads of stage cl
    // into slot sl, all interleaved with the MFMA groups (one group = the TM blocks of one jn).
    // TNX = the wave's number of 32-column blocks (TN, or TN_LAST in the last wave column).
    // (sb / sbn: B slots of this and the next stage -- s / sn unless the ring is split -- and, split,
    // B stage cl + 1 goes to B slot sb)
    auto compute = [&](int s, auto u_tag, auto buf_tag, auto loads_tag, auto tnx_tag, int sn, int cl, int sl,
                       bool load_live, int sb, int sbn, bool load_live_b) {
        constexpr int u = decltype(u_tag)::value;
        constexpr int buf = decltype(buf_tag)::value;
        // loads_tag: bit 0 = this wave issues global->LDS loads, bit 1 = its rows are all past the
        // group's valid rows (anchored tiles): it keeps the ring's loads and barriers, no MFMAs
        constexpr bool kLoadWave = (decltype(loads_tag)::value & 1) != 0;
        constexpr bool kDeadRows = (decltype(loads_tag)::value & 2) != 0;
        constexpr bool kLoads = kLoadWave && u == 0 && (!kLate || kSpread);
        constexpr int TNX = decltype(tnx_tag)::value;
        constexpr int kLPG = (NL + TNX - 1) / TNX;
        constexpr bool kAhead = u + 1 < KM || kCross;
        const uint8_t* sB = b_slot(sb);
        const uint8_t* sSB = a_slot(s) + SC_OFF + u * SCU + SCA;
        i32x8 fb_cur = fb0[buf];
        int sb_cur = sb0[buf];
        static_for<TNX>([&](auto jn_c) {
            constexpr int jn = decltype(jn_c)::value;
            i32x8 fb_next = fb_cur;
            int sb_next = sb_cur;
            if constexpr (jn + 1 < TNX) {
                if constexpr (BMN) fb_next = load_frag_mn(sB, wn * WN + (jn + 1) * 32, u_tag);
                else fb_next = load_frag(sB, wn * WN + (jn + 1) * 32 + r, Int<SPRB>{}, u_tag);
                if constexpr (!kBf16) sb_next = load_scale(sSB, wn * WN + (jn + 1) * 32 + r);
            }
            if constexpr (kLate && u + 1 == KM && jn + 1 == TNX) {
                // late sync: this stage's slot s is no longer read by anyone after the barrier
                // and stage cl - 1 has landed; refill s with stage cl and read stage cl - 1's
                // first fragments (slot sn) into the sub-step-0 registers
                // (split ring: B of stage cl - 1, issued at the previous sync after A / SF of stage
                // cl - 1, may stay in flight)
                wait_vmcnt<kSplitRing ? kMinLoadsB : 0>();
                stage_barrier();
                static_for<TM + 1>([&](auto part_c) { prefetch(sn, sbn, Int<0>{}, part_c, Int<0>{}); });
                // (the reads go out before this group's MFMAs, which then cover their latency)
                __builtin_amdgcn_sched_barrier(0);
                if constexpr (kLoadWave && !kSpread) {
                    if constexpr (kSplitRing) issue_split(cl, sl, load_live, cl + 1, sb, load_live_b);
                    else issue_stage(cl, sl, load_live);
                }
            }
            static_for<TM>([&](auto jm_c) {
                constexpr int jm = decltype(jm_c)::value;
                if constexpr (kDeadRows) {
                } else if constexpr (kBf16) {
                    const i32x4 b0 = {fb_cur[0], fb_cur[1], fb_cur[2], fb_cur[3]};
                    const i32x4 b1 = {fb_cur[4], fb_cur[5], fb_cur[6], fb_cur[7]};
                    const i32x4 a0 = {fa[buf][jm][0], fa[buf][jm][1], fa[buf][jm][2], fa[buf][jm][3]};
                    const i32x4 a1 = {fa[buf][jm][4], fa[buf][jm][5], fa[buf][jm][6], fa[buf][jm][7]};
                    acc[jn][jm] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                        __builtin_bit_cast(bf16x8, b0), __builtin_bit_cast(bf16x8, a0), acc[jn][jm], 0, 0, 0);
                    acc[jn][jm] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                        __builtin_bit_cast(bf16x8, b1), __builtin_bit_cast(bf16x8, a1), acc[jn][jm], 0, 0, 0);
                } else {
                    acc[jn][jm] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
                        fb_cur, fa[buf][jm], acc[jn][jm], kFmtB, kFmtA, 0, sb_cur, 0, sa[buf][jm]);
                }
            });
            // ahead registers of the next sub-step: A block jm goes with group jm * TNX / TM, the
            // first B block with the last group (a cross-stage read of slot sn past the last
            // stage reads stale bytes that are never used)
            if constexpr (kAhead) {
                static_for<TM + 1>([&](auto part_c) {
                    constexpr int part = decltype(part_c)::value;
                    constexpr int grp = part < TM ? part * TNX / TM : TNX - 1;
                    if constexpr (grp == jn) {
                        if constexpr (u + 1 < KM) prefetch(s, sb, Int<buf ^ 1>{}, Int<part>{}, Int<u + 1>{});
                        else prefetch(sn, sbn, Int<buf ^ 1>{}, Int<part>{}, Int<0>{});
                    }
                });
            }
            static_for<kLPG>([&](auto li) {
                constexpr int idx = jn * kLPG + decltype(li)::value;
                if constexpr (kLoads && idx < NL) issue_item(Int<idx>{}, cl, sl, load_live);
            });
            __builtin_amdgcn_sched_barrier(0);
            fb_cur = fb_next;
            sb_cur = sb_next;
        });
    };

    // ------------------------------------------------------------------ main loop
    // Prologue: stages 0 .. NSTAGE-2 in flight; with a cross-stage ring, stage 0 visible and its
    // ahead registers loaded.
    // (A two-slot ring fills both slots.)
    constexpr int kPro = kLate && !kSpread ? 2 : NSTAGE - 1;
    static_for<kPro>([&](auto i) {
        constexpr int st = decltype(i)::value;
        if (is_loader) issue_stage(c0 + st - shift, st, st >= shift && st < num_virtual);
    });
    if constexpr (kSplitRing) {
        // (split ring: B of stage 2 into B slot 2 as well; stages 0 and 1 went out whole)
        if (is_loader)
            static_for<NLB>([&](auto i) { issue_item(Int<NLA + decltype(i)::value>{}, c0 + 2, 2, 2 < num_virtual); });
    }
    if constexpr (kCross || kLate) {
        wait_vmcnt<(kPro - 1) * kMinLoadsPerStage + (kSplitRing ? kMinLoadsB : 0)>();
        stage_barrier();
        static_for<TM + 1>([&](auto part_c) { prefetch(0, 0, Int<0>{}, part_c, Int<0>{}); });
    }

    // Cross-stage ring: stage c + 1 must have landed before the barrier of iteration c (its ahead
    // registers are read during stage c); the loads of stages c + 2 .. c + NSTAGE - 2 may stay in
    // flight.  The barrier also certifies that every wave finished reading stage c - 1 (its B
    // side in iteration c - 1, its ahead registers in iteration c - 2), so its slot can take
    // stage c + NSTAGE - 1.  Otherwise stage c must have landed (stages c + 1 .. c + NSTAGE - 2
    // may be in flight), the barrier certifies that stage c - 1 is no longer read, and the
    // stage's first fragments are read after it.  A late-sync ring has no barrier here: it met
    // before the previous stage's last MFMA group (see compute).
    auto iteration = [&](int c, auto pbuf_tag, auto loads_tag, auto tnx_tag) {
        if constexpr (!kLate) {
            wait_vmcnt<(NSTAGE - (kCross ? 3 : 2)) * kMinLoadsPerStage>();
            stage_barrier();
        }
        const int cl = c + (kLate && !kSpread ? 2 : NSTAGE - 1);
        constexpr int buf0 = KM == 1 ? decltype(pbuf_tag)::value : 0;
        if constexpr (!kCross && !kLate)
            static_for<TM + 1>([&](auto part_c) { prefetch(c % NSTAGE, c % NSTAGE, Int<buf0>{}, part_c, Int<0>{}); });
        static_for<KM>([&](auto u_c) {
            constexpr int u = decltype(u_c)::value;
            constexpr int buf = KM == 1 ? decltype(pbuf_tag)::value : u;
            compute(c % NSTAGE, u_c, Int<buf>{}, loads_tag, tnx_tag, (c + 1) % NSTAGE, c0 + cl - shift, cl % NSTAGE,
                    cl < num_virtual, c % NSB, (c + 1) % NSB, cl + 1 < num_virtual);
        });
    };
    // Loader and non-loader waves run separate copies of the loop, each branch-free.
    auto main_loop = [&](auto loads_tag, auto tnx_tag) {
        if constexpr (KM == 1) {
            for (int c = 0; c < num_virtual; c += 2) {
                iteration(c, Int<0>{}, loads_tag, tnx_tag);
                iteration(c + 1, Int<1>{}, loads_tag, tnx_tag);
            }
        } else {
            for (int c = 0; c < num_virtual; ++c) iteration(c, Int<0>{}, loads_tag, tnx_tag);
        }
    };
    // (anchored tiles: a wave whose rows all lie past the group's valid rows runs a copy of the
    // loop without MFMAs; its accumulators stay zero)
    const bool dead_rows = BM > 256 && m0 + wm * WM >= valid_end;
    if constexpr (BM > 256) {
        if (dead_rows) {
            if (LW == NW || is_loader) main_loop(Int<3>{}, Int<TN_LAST>{});
            else main_loop(Int<2>{}, Int<TN>{});
        } else {
            if (LW == NW || is_loader) main_loop(Int<1>{}, Int<TN_LAST>{});
            else main_loop(Int<0>{}, Int<TN>{});
        }
    } else {
        if (LW == NW || is_loader) main_loop(Int<1>{}, Int<TN_LAST>{});   // loaders = the last wave column
        else main_loop(Int<0>{}, Int<TN>{});
    }
    __builtin_amdgcn_s_waitcnt(0);

    // ------------------------------------------------------------------ split-K reduction
    if (!kRagged && split_k > 1) {   // (the host never splits a ragged tile)
        // This workgroup's partial tile, in accumulator-register order (coalesced 16-byte
        // stores and loads; the reducing workgroup uses the same lane mapping).
        // Lanes of rows past M (skinny M) take an offset past the buffer's end: the hardware
        // drops their stores and returns zeros for their loads, so no partial bytes move for them.
        float* const tile_ws = p.ws + (int64_t)tile_id * split_k * (BM * BN);
        const __amdgpu_buffer_rsrc_t rs_ws = make_rsrc(tile_ws, (int64_t)split_k * (BM * BN) * 4);
        auto part_off = [&](int sp, int jn, int jm) -> uint32_t {
            const int m = m0 + wm * WM + jm * 32 + r;
            return m < M ? (uint32_t)(sp * (BM * BN) + (((wave * TN + jn) * TM + jm) * 64 + lane) * 16) * 4u
                         : 0x80000000u;
        };
        static_for<TN>([&](auto jn_c) {
            constexpr int jn = decltype(jn_c)::value;
            static_for<TM>([&](auto jm_c) {
                constexpr int jm = decltype(jm_c)::value;
                const uint32_t off = part_off(split, jn, jm);
#pragma unroll
                for (int g = 0; g < 4; ++g)
                    __builtin_amdgcn_raw_buffer_store_b128(
                        __builtin_bit_cast(u32x4, f32x4{acc[jn][jm][4 * g], acc[jn][jm][4 * g + 1], acc[jn][jm][4 * g + 2],
                                                        acc[jn][jm][4 * g + 3]}),
                        rs_ws, off + 16 * g, 0, kCacheSc1);
            });
        });
        // Publish the partial and count arrivals; only the last workgroup of the tile goes on.
        // The partials are stored and reloaded at device scope (written through to memory, read
        // coherently on every XCD), so once every wave's stores are acknowledged they are
        // visible to whichever workgroup reduces, on whichever XCD, and no fence (an L2
        // writeback or invalidate) is needed.  The "memory" clobber keeps the compiler from
        // sinking the stores past the wait.  This follows the GFX942 code sequences of the LLVM
        // AMDGPU memory model (llvm/docs/AMDGPUUsage.rst, "Memory Model GFX942", which gfx950
        // shares): a monotonic agent-scope atomic store or load is a plain buffer store / load
        // with sc1 set, so these partial stores and loads are relaxed agent-scope atomics; an
        // agent-scope release is "buffer_wbl2 sc1=1; s_waitcnt vmcnt(0)", whose L2 writeback
        // serves only non-atomic data, so the vmcnt(0) before the counter's fetch-add is the whole
        // release here; the acquire's "buffer_inv sc1=1" likewise serves only non-atomic loads,
        // so the reducing workgroup's sc1 loads need none.  (tests/test_split_k_gpu.py forces the
        // splits of one tile onto different XCDs to keep this checked.)
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        int* flag = reinterpret_cast<int*>(smem);
        if (tid == 0)
            *flag = __hip_atomic_fetch_add(p.counters + tile_id, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __syncthreads();
        if (*flag != split_k - 1) return;
        // Sum the partials in split order, whichever split arrived last, so a launch's result
        // does not depend on workgroup timing.  Small wave tiles keep the loads of partial sp + 1
        // in flight while partial sp is added (two register sets), so the reduction costs about
        // one L2 round trip instead of split_k of them.
        static_for<TN>([&](auto i) {
            static_for<TM>([&](auto j) { acc[decltype(i)::value][decltype(j)::value] = f32x16{}; });
        });
        f32x4 pb[TM * TN <= 4 ? 2 : 1][TN][TM][4];
        auto load_part = [&](int sp, auto set_tag) {
            constexpr int set = decltype(set_tag)::value;
            static_for<TN>([&](auto jn_c) {
                constexpr int jn = decltype(jn_c)::value;
                static_for<TM>([&](auto jm_c) {
                    constexpr int jm = decltype(jm_c)::value;
                    // device-scope loads: coherent with the device-scope partial stores
                    const uint32_t off = part_off(sp, jn, jm);
#pragma unroll
                    for (int g = 0; g < 4; ++g)
                        pb[set][jn][jm][g] = __builtin_bit_cast(
                            f32x4, __builtin_amdgcn_raw_buffer_load_b128(rs_ws, off + 16 * g, 0, kCacheSc1));
                });
            });
        };
        auto add_part = [&](auto set_tag) {
            constexpr int set = decltype(set_tag)::value;
            static_for<TN>([&](auto jn_c) {
                constexpr int jn = decltype(jn_c)::value;
                static_for<TM>([&](auto jm_c) {
                    constexpr int jm = decltype(jm_c)::value;
#pragma unroll
                    for (int g = 0; g < 4; ++g)
#pragma unroll
                        for (int i = 0; i < 4; ++i) acc[jn][jm][4 * g + i] += pb[set][jn][jm][g][i];
                });
            });
        };
        if constexpr (TM * TN <= 4) {
            // (a partial index past the last one re-reads partial 0: in range, never added)
            load_part(0, Int<0>{});
            for (int sp = 0; sp < split_k; sp += 2) {
                load_part(sp + 1 < split_k ? sp + 1 : 0, Int<1>{});
                add_part(Int<0>{});
                load_part(sp + 2 < split_k ? sp + 2 : 0, Int<0>{});
                if (sp + 1 < split_k) add_part(Int<1>{});
            }
        } else {
            // (large wave tiles: no registers for a second set)
            for (int sp = 0; sp < split_k; ++sp) {
                load_part(sp, Int<0>{});
                add_part(Int<0>{});
            }
        }
        if (tid == 0) __hip_atomic_store(p.counters + tile_id, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }

    // ------------------------------------------------------------------ epilogue
    // All accumulator indexing is in compile-time-unrolled loops (static_for): a runtime
    // index would demote the accumulator array to scratch memory.
    static_for<TM>([&](auto jm_c) {
        constexpr int jm = decltype(jm_c)::value;
        const int m = m0 + wm * WM + jm * 32 + r;
        const bool row_ok = m < tile_end && !(gemm_type == kMasked && m >= valid_end);
        bool pad_row = false;
        if (gemm_type == kMGroupedPsum) pad_row = m >= valid_end;
        // (an anchored m_indices tile knows its run's valid end: the checked layout holds one group on a
        // prefix of each alignment block, so no row id needs reading)
        else if (gemm_type == kMGroupedIdx) pad_row = anchored ? m >= valid_end : row_ok && p.layout[m] != group;
        if constexpr (EPI == kEpiF32 || EPI == kEpiBf16) {
            if (p.accumulate) {
                // the old D of this row of blocks in one burst, then the blocks
                float old[TN][16];
                static_for<TN>([&](auto jn_c) {
                    constexpr int jn = decltype(jn_c)::value;
                    if (!(kRagged && jn >= TN_LAST && wn == WGN - 1))
                        load_old_block<EPI>(p, d_base, m, row_ok, n0 + wn * WN + jn * 32, N, q, old[jn]);
                });
                static_for<TN>([&](auto jn_c) {
                    constexpr int jn = decltype(jn_c)::value;
                    if (kRagged && jn >= TN_LAST && wn == WGN - 1) return;
                    epilogue_block<EPI>(p, acc[jn][jm], d_base, m, row_ok, pad_row, n0 + wn * WN + jn * 32, N, batch, q,
                                        old[jn]);
                });
                return;
            }
        }
        static_for<TN>([&](auto jn_c) {
            constexpr int jn = decltype(jn_c)::value;
            if (kRagged && jn >= TN_LAST && wn == WGN - 1) return;   // no such block in this wave
            epilogue_block<EPI>(p, acc[jn][jm], d_base, m, row_ok, pad_row, n0 + wn * WN + jn * 32, N, batch, q);
        });
    });
}

// Persistent walk over the real tiles of an anchored M-grouped launch (the reference's psum
// scheduler, deep_gemm/include/deep_gemm/scheduler.hpp:144-162, on CDNA4 terms): one workgroup
// per CU counts the layout's tiles once and serves tiles b, b + gridDim.x, ... below that count,
// instead of a grid sized for the worst case whose spare workgroups exit.
template <int BM, int BN, int WGM, int NW, int LW, int NSTAGE, int KM, int OCC, int KIND, int EPI, int NSB = 0>
__global__ __launch_bounds__(NW * 64, OCC * NW / 4) void gemm_walk_kernel(const KParams p) {
    const int gemm_type = p.gemm_type;
    const int* runs = gemm_type == kMGroupedIdx ? p.runs : nullptr;
    const int total = __builtin_amdgcn_readfirstlane(
        anchored_total(p.layout, p.num_groups, runs, p.alignment, BM, p.m, p.num_n_blocks));
    for (int vb = blockIdx.x; vb < total; vb += gridDim.x) {
        gemm_body<BM, BN, WGM, NW, LW, NSTAGE, KM, OCC, KIND, EPI, -1, 0, 0, 0, 0, false, false, NSB>(p, vb, total);
        // (every load of the tile, including the ring's dead ones, lands before the next tile's)
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
    }
}

// The ahead-of-time kernel of one tile shape: everything from the arguments.
template <int BM, int BN, int WGM, int NW, int LW, int NSTAGE, int KM, int OCC, int KIND, int EPI, bool AMN = false,
          bool BMN = false, int NSB = 0>
__global__ __launch_bounds__(NW * 64, OCC * NW / 4) void gemm_kernel(const KParams p) {
    gemm_body<BM, BN, WGM, NW, LW, NSTAGE, KM, OCC, KIND, EPI, -1, 0, 0, 0, 0, AMN, BMN, NSB>(p, blockIdx.x + p.vbase);
}

}  // namespace dg
