// Decode GEMV kernel for gfx950: e4m3 x e4m3 GEMMs with M <= 4 rows (dense or batched).
//
// At M <= 4 a GEMM is a read of B (N x K bytes) and little else.  The MFMA decode kernels spend
// their time on fixed costs around that read (a chain of group-sized round trips per wave, and a
// split-K partial store / count / reload across workgroups when the strips alone do not fill the
// CUs).  Here the arithmetic runs on the VALU and K is split only between the waves of one
// workgroup:
//
// * B is read in groups of 8 rows: one load instruction of a wave moves 8 rows x 128 bytes
//   (lane l: row l / 8, bytes 16 (l % 8) .. + 16 of the step's 128-byte column), the load shape
//   that measured fastest from HBM on this part (a wave streaming 1 KB of one row per
//   instruction ran at 3.8 TB/s on 7168x16384 without any arithmetic).  A lane keeps its row for
//   the whole kernel, so its accumulator belongs to one row;
// * a workgroup of NWV = 8 or 4 waves owns 8 NWV / ks rows: wave w takes row group w / ks and the (w % ks)-th of
//   ks contiguous K ranges of it, DP steps (1 KB each) in flight, straight into registers; the
//   packed scale int16 of the lane's 64-K block comes with each step;
// * A (M rows, at most ~60 KB as f16) is converted once per workgroup into LDS as f16 (e4m3 ->
//   f16 is exact: 448 and 2^-9 are f16 normals), with its UE8M0 scale bytes beside it;
// * a step's 16 B values per lane become f16 pairs with v_cvt_scalef32_pk_f16_fp8 (scale 1:
//   exact) and meet A in v_dot2c_f32_f16 (exact products, fp32 sums); the 16-element dot is
//   scaled by 2^(sa + sb - 254) (v_ldexp_f32, the per-32-K UE8M0 pair of the MFMA recipe) and
//   added to the lane's accumulator;
// * at the end the 8 lanes of a row are summed in a fixed butterfly, the K ranges' sums meet in
//   LDS and are added in range order (deterministic), and one thread per row of D applies the
//   epilogue (alpha, bias, accumulate, bf16 RNE or fp32).
//
// ks (KParams::split_stages) and the number of workgroups per batch (KParams::num_n_blocks) come
// from the host; workgroups are dealt over the 8 XCDs in contiguous runs so that neighbouring row
// groups (which share the scale rows' cache lines) share an L2.
#include "gemm_kernel.hpp"
#include "gemm_tiles.hpp"
#include "skinny_kernel.hpp"

namespace dg {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
struct __attribute__((aligned(32))) h2x8 {
    h2 v[8];
};

// 16 e4m3 values (4 dwords, byte i = element i) -> 8 f16 pairs, exactly (scale 1; every e4m3 value
// is an f16 normal or zero).
__device__ __forceinline__ void fp8x16_to_f16(const i32x4 x, h2* h) {
#pragma unroll
    for (int d = 0; d < 4; ++d) {
        h[2 * d] = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8((uint32_t)x[d], 1.0f, false);
        h[2 * d + 1] = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8((uint32_t)x[d], 1.0f, true);
    }
}

// Steps in flight per wave.  Six keep M <= 2 within 64 VGPRs (eight waves per SIMD, so that every
// workgroup of a launch fits one round: 1x24576x1536 10.0 vs 11.0 us with eight steps at 73 VGPRs,
// the other decode shapes level).
constexpr int kGemvDepth = 6;

// LDS bytes of one workgroup: A as f16 [MR][kp], A's scale bytes [MR][kp / 32], the K ranges'
// row sums [MR][8 NWV / ks][ks] (at most MR x 64 floats)
__host__ __device__ constexpr int gemv_kp(int k) { return (k + 127) / 128 * 128; }
inline int gemv_lds_bytes(int mr, int k, int /*ks*/) { return mr * gemv_kp(k) * 2 + mr * gemv_kp(k) / 32 + mr * 64 * 4; }

template <int MR, int EPI, int NWV>
__device__ __forceinline__ void gemv_body(const KParams& p, const int vb) {
    constexpr int DP = kGemvDepth;
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int K = p.k, kp = gemv_kp(K), N = p.n;
    const int ks = p.split_stages, rows_wg = 8 * NWV / ks;
    _Float16* const a_lds = reinterpret_cast<_Float16*>(smem);              // [MR][kp]
    uint8_t* const sa_lds = smem + MR * kp * 2;                              // [MR][kp / 32]
    float* const part_lds = reinterpret_cast<float*>(sa_lds + MR * kp / 32);  // [MR][rows_wg][ks]

    // workgroup of this block: contiguous runs of workgroups per XCD (block b runs on XCD b % 8)
    const int wgs = p.num_tiles, per_xcd = ceil_div(wgs, 8);
    const int c = (vb % 8) * per_xcd + vb / 8;
    if (c >= wgs) return;
    const int batch = c / p.num_n_blocks;
    const int n0 = (c - batch * p.num_n_blocks) * rows_wg;
    const uint8_t* a_base = p.a;
    const uint8_t* b_base = p.b;
    const uint16_t* sfa = p.sfa;
    const uint16_t* sfb = p.sfb;
    uint8_t* d_base = p.d;
    if (p.gemm_type == kBatched) {
        a_base += (int64_t)batch * p.bsa;
        b_base += (int64_t)batch * p.bsb;
        sfa += (int64_t)batch * p.sfa_bs;
        sfb += (int64_t)batch * p.sfb_bs;
        d_base += (int64_t)batch * p.bsd * p.out_esize;
    }
    const int M = p.m;
    const int nk64 = ceil_div(K, 64);
    const int kbytes = p.kbytes_b;   // == K for e4m3

    // ------------------------------------------------------------------ B stream set-up
    const int grp = w / ks, split = w - grp * ks;              // row group and K range of this wave
    const int r = lane >> 3, cb = (lane & 7) * 16;             // lane's row in the group, byte in a step
    const int row = grp * 8 + r;                               // row in the workgroup
    const bool row_ok = n0 + row < N;
    const int pk = kp / 128;                                   // 128-byte steps of a row
    const int spw = ceil_div(pk, ks);                          // steps of a K range
    const int st0 = split * spw, st1 = min(pk, st0 + spw);
    const int rows_b = max(0, min(rows_wg, N - n0));
    const __amdgpu_buffer_rsrc_t rs_b = make_rsrc(b_base + (int64_t)n0 * p.ldb, (int64_t)rows_b * p.ldb);
    const __amdgpu_buffer_rsrc_t rs_sb = make_rsrc(sfb, (int64_t)nk64 * p.sfb_ld * 2);
    const int ldb = (int)p.ldb;
    const int sfb_step = (int)p.sfb_ld * 2;
    const uint32_t vrow = (uint32_t)(row * ldb + cb);
    const uint32_t vsrow = (uint32_t)((((n0 + row) & ~1) * 2) + (cb >> 6) * sfb_step);
    i32x4 buf[DP];
    uint32_t sbuf[DP];
    int lst = st0;   // step loaded next
    auto issue = [&](auto slot_tag) {
        constexpr int j = decltype(slot_tag)::value;
        const bool on = row_ok && lst < st1 && lst * 128 + cb < kbytes;
        // (offsets computed unconditionally and pinned, so that the compiler selects them rather
        // than branching around the loads, which cost it its wait counting)
        uint32_t v = vrow + (uint32_t)(lst * 128);
        uint32_t vs = vsrow + (uint32_t)(lst * 2 * sfb_step);
        asm volatile("" : "+v"(v), "+v"(vs));
        v = on ? v : kOOBOffset;
        vs = on ? vs : kOOBOffset;
        buf[j] = __builtin_bit_cast(i32x4, __builtin_amdgcn_raw_buffer_load_b128(rs_b, v, 0, 0));
        // (the aligned dword holding the packed pairs of rows 2i and 2i + 1: a 16-bit load's
        // zero-extension gets hoisted by the compiler to where it waits for every load in flight)
        sbuf[j] = __builtin_amdgcn_raw_buffer_load_b32(rs_sb, vs, 0, 0);
        ++lst;
    };

    // ------------------------------------------------------------------ A -> LDS as f16
    // (each thread's first A piece and scale pair are loaded before B's first steps are issued,
    // so that waiting for them does not wait for B)
    const __amdgpu_buffer_rsrc_t rs_a = make_rsrc(a_base, (int64_t)M * p.lda);
    const __amdgpu_buffer_rsrc_t rs_sa = make_rsrc(sfa, (int64_t)nk64 * p.sfa_ld * 2);
    const int pieces = kp / 16, kb64 = kp / 64;
    auto a_offset = [&](int i) -> uint32_t {
        const int m = i / pieces, kofs = (i - m * pieces) * 16;
        return m < M && kofs < kbytes ? (uint32_t)(m * p.lda + kofs) : kOOBOffset;
    };
    auto sa_offset = [&](int i) -> uint32_t {
        const int m = i / kb64, kb = i - m * kb64;
        return m < M && kb < nk64 ? (uint32_t)((kb * p.sfa_ld + m) * 2) : kOOBOffset;
    };
    auto a_store = [&](int i, const i32x4 x) {
        const int m = i / pieces, kofs = (i - m * pieces) * 16;
        h2 h[8];
        fp8x16_to_f16(x, h);
        i32x4* dst = reinterpret_cast<i32x4*>(a_lds + m * kp + kofs);
        dst[0] = i32x4{__builtin_bit_cast(int, h[0]), __builtin_bit_cast(int, h[1]), __builtin_bit_cast(int, h[2]),
                       __builtin_bit_cast(int, h[3])};
        dst[1] = i32x4{__builtin_bit_cast(int, h[4]), __builtin_bit_cast(int, h[5]), __builtin_bit_cast(int, h[6]),
                       __builtin_bit_cast(int, h[7])};
    };
    // scale bytes: sa_lds[m][2 kb + h] = byte h of the packed int16 of (row m, 64-K block kb)
    auto sa_store = [&](int i, uint32_t s) {
        const int m = i / kb64, kb = i - m * kb64;
        sa_lds[m * (kp / 32) + 2 * kb] = (uint8_t)(s & 0xff);
        sa_lds[m * (kp / 32) + 2 * kb + 1] = (uint8_t)(s >> 8);
    };
    constexpr int T = NWV * 64;
    const bool a0_on = tid < MR * pieces, s0_on = tid < MR * kb64;
    const i32x4 x0 = __builtin_bit_cast(i32x4, __builtin_amdgcn_raw_buffer_load_b128(rs_a, a0_on ? a_offset(tid) : kOOBOffset, 0, 0));
    const uint32_t sx0 = __builtin_amdgcn_raw_buffer_load_b16(rs_sa, s0_on ? sa_offset(tid) : kOOBOffset, 0, 0);

    static_for<DP>([&](auto j) { issue(j); });

    if (a0_on) a_store(tid, x0);
    if (s0_on) sa_store(tid, sx0);
    for (int i = tid + T; i < MR * pieces; i += T)
        a_store(i, __builtin_bit_cast(i32x4, __builtin_amdgcn_raw_buffer_load_b128(rs_a, a_offset(i), 0, 0)));
    for (int i = tid + T; i < MR * kb64; i += T) sa_store(i, __builtin_amdgcn_raw_buffer_load_b16(rs_sa, sa_offset(i), 0, 0));
    __syncthreads();

    // ------------------------------------------------------------------ main loop
    float acc[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) acc[m] = 0.f;
    // byte (row % 2) * 2 + half of the scale dword: the lane's 32-K half of its 64-K block
    const int ssh = ((cb >> 5) & 1) * 8 + ((n0 + row) & 1) * 16;
    int cst = st0;   // step computed next
    auto compute = [&](auto slot_tag) {
        constexpr int j = decltype(slot_tag)::value;
        const i32x4 x = buf[j];
        h2 hb[8];
        fp8x16_to_f16(x, hb);
        // (a step past the range holds zeros; its A reads stay inside the row)
        const int kofs = min(cst, pk - 1) * 128 + cb;
        const int sb = shift_at_use((int)sbuf[j], ssh) & 0xff;
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            // 32 bytes, 32-aligned, read as f16 pairs (read as i32x4 halves with a bit cast per
            // element, the compiler fed the first dword of each half to all four dots)
            const h2x8 av = *reinterpret_cast<const h2x8*>(a_lds + m * kp + kofs);
            float dot = 0.f;
#pragma unroll
            for (int d = 0; d < 8; ++d) dot = __builtin_amdgcn_fdot2(hb[d], av.v[d], dot, false);
            const int sa = sa_lds[m * (kp / 32) + (kofs >> 5)];
            acc[m] += __builtin_amdgcn_ldexpf(dot, sa + sb - 254);
            // (pinned here: otherwise the compiler sinks every slot's arithmetic below the pass's
            // last load, keeping all eight steps' data live: 170-256 registers)
            asm volatile("" : "+v"(acc[m]));
        }
        ++cst;
    };
    // Every slot computes and reloads on every pass, with no branch around the loads (steps past
    // the range load nothing and add zeros), so the compiler's count of the loads in flight is the
    // same on every path and each slot waits only for its own step.
    for (int s0 = st0; s0 < st1; s0 += DP) {
        static_for<DP>([&](auto j_c) {
            compute(j_c);
            issue(j_c);
        });
    }
    // the 8 lanes of a row, then the K ranges of the row in LDS
#pragma unroll
    for (int m = 0; m < MR; ++m) {
        float v = acc[m];
        v += __shfl_xor(v, 1, 64);
        v += __shfl_xor(v, 2, 64);
        v += __shfl_xor(v, 4, 64);
        if ((lane & 7) == 0) part_lds[(m * rows_wg + row) * ks + split] = v;
    }
    __syncthreads();

    // ------------------------------------------------------------------ epilogue: D rows
    constexpr bool kF32 = EPI == kEpiF32;
    using OutT = typename Cond<kF32, float, uint16_t>::type;
    const OutT* bp = reinterpret_cast<const OutT*>(p.bias);
    auto to_f = [](OutT x) -> float {
        if constexpr (kF32) return x; else return bf16_to_f32(x);
    };
    for (int i = tid; i < MR * rows_wg; i += T) {
        const int m = i / rows_wg, rr = i - m * rows_wg;
        if (m >= M || rr >= rows_b) continue;
        const int n = n0 + rr;
        OutT* dp = reinterpret_cast<OutT*>(d_base) + (int64_t)m * p.ldd + n;
        const float* pr = part_lds + (m * rows_wg + rr) * ks;
        float v = 0.f;
        for (int l = 0; l < ks; ++l) v += pr[l];   // (K ranges in order: deterministic)
        v *= p.alpha;
        if (p.has_bias) v += to_f(bp[n]);
        if (p.accumulate) v += to_f(*dp);
        if constexpr (kF32) *dp = v; else *dp = f32_to_bf16_rne(v);
    }
}

template <int MR, int EPI, int NWV>
__global__ __launch_bounds__(NWV * 64, MR <= 2 ? 8 : 4) void gemv_kernel(const KParams p) {
    gemv_body<MR, EPI, NWV>(p, blockIdx.x + p.vbase);
}

template <int MR, int NWV>
KernelFn gemv_epi(int epi) {
    return epi == kEpiF32 ? &gemv_kernel<MR, kEpiF32, NWV> : epi == kEpiBf16 ? &gemv_kernel<MR, kEpiBf16, NWV> : nullptr;
}

KernelFn lookup_gemv(int mr, int epi, int waves) {
    if (waves != 4 && waves != 8) return nullptr;
    const bool w8 = waves == 8;
    switch (mr) {
        case 1: return w8 ? gemv_epi<1, 8>(epi) : gemv_epi<1, 4>(epi);
        case 2: return w8 ? gemv_epi<2, 8>(epi) : gemv_epi<2, 4>(epi);
        case 4: return w8 ? gemv_epi<4, 8>(epi) : gemv_epi<4, 4>(epi);
        default: return nullptr;
    }
}

int gemv_lds(int mr, int k, int ks) { return gemv_lds_bytes(mr, k, ks); }

}  // namespace dg
