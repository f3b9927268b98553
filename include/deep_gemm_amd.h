/*
 * deep_gemm_amd.h -- C ABI of the MI355X (gfx950) block-scaled GEMM library
 * (libdeep_gemm_amd.so).  Plain pointers, sizes and strides only; no torch types.
 *
 * All device pointers are HIP device addresses; `stream` is a hipStream_t (NULL = the
 * default stream).  Every entry point is asynchronous on `stream` and returns 0 on success
 * or a negative DG_E* code; dg_last_error() then holds a message (thread-local).
 *
 * Scale factors (SF) consumed by the GEMM entry points are in the "required layout" that
 * dg_transform_sf() produces, which is the layout the reference documents for
 * transform_sf_into_required_layout (csrc/apis/layout.hpp:18-35): one UE8M0 exponent byte
 * per 32 K-elements, two K-adjacent bytes per int16 (even block in the low byte), stored
 * MN-major: element (mn, k64) at sf[k64 * sf_ld + mn], with sf_ld (and any batch stride)
 * even -- the kernels fetch SF rows two at a time.
 */
#ifndef DEEP_GEMM_AMD_H_
#define DEEP_GEMM_AMD_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Operand format pairs (A x B). */
#define DG_KIND_FP8_FP8   0   /* e4m3 x e4m3, per-32 UE8M0 scales on both operands          */
#define DG_KIND_FP8_FP4   1   /* e4m3 x e2m1 (B packed two per byte, low nibble = even k)   */
#define DG_KIND_FP4_FP4   2   /* e2m1 x e2m1                                                 */
#define DG_KIND_BF16      3   /* bf16 x bf16, no scales                                      */

/* Work decomposition. */
#define DG_GEMM_NORMAL        0  /* D[M,N] = A[M,K] B[N,K]^T                                  */
#define DG_GEMM_BATCHED       1  /* D[g] = A[g] B[g]^T for g < num_groups                     */
#define DG_GEMM_MGROUPED_PSUM 2  /* grouped_layout = psum int32[G]; group g = rows
                                    [align(psum[g-1], alignment), psum[g]) uses B[g]          */
#define DG_GEMM_MGROUPED_IDX  3  /* grouped_layout = m_indices int32[M]; -1 marks padding rows */
#define DG_GEMM_MASKED        4  /* A[G,M,K], D[G,M,N]; grouped_layout = masked_m int32[G]     */
#define DG_GEMM_KGROUPED      5  /* A[M,Ktot], B[N,Ktot] (K-major), D[G,M,N]; grouped_layout =
                                    psum int32[G] over K; group g contracts K
                                    [align(psum[g-1], alignment), psum[g]) into D[g]
                                    (k_grouped_fp8_gemm_tn_contiguous, csrc/apis/gemm.hpp:351-387);
                                    alignment a multiple of 64; accumulate allowed              */

#define DG_DTYPE_BF16     0
#define DG_DTYPE_F32      1
#define DG_DTYPE_FP8_E4M3 2   /* e4m3 D quantised per (row, 32 columns) with UE8M0 scales in sfd
                                 (the FP8Quantization epilogue, csrc/jit_kernels/epilogue_class.hpp:77-107,
                                 deep_gemm/include/deep_gemm/epilogue/operators.hpp:339-463):
                                 DG_KIND_FP8_FP8, DG_GEMM_NORMAL / BATCHED, n % 128 == 0, no
                                 accumulate / bias / alpha                                       */

/* Output rounding of a bf16 D. */
#define DG_EPI_DEFAULT 0      /* round to nearest even                                          */
#define DG_EPI_BF16_SR 1      /* stochastic rounding keyed by a hash of each quartet of fp32
                                 outputs (the BF16StochasticRounding epilogue,
                                 deep_gemm/include/deep_gemm/epilogue/operators.hpp:224-337);
                                 bf16 D, no accumulate / bias / alpha                           */

#define DG_SF_F32 0   /* fp32 powers of two, one per gran_mn x gran_k block             */
#define DG_SF_I16 1   /* packed UE8M0x2 int16, one per gran_mn x 64                       */

#define DG_OK            0
#define DG_EINVAL       -1   /* invalid argument / unsupported shape or layout           */
#define DG_ELAUNCH      -2   /* HIP launch error                                           */
#define DG_ENOKERNEL    -3   /* no compiled kernel for the requested configuration         */

/*
 * Problem description for dg_gemm().  Replaces the reference's GemmDesc
 * (csrc/jit_kernels/gemm_config.hpp:39-95) as the argument of launch_fp8_gemm /
 * launch_fp4_gemm / launch_fp8_dequant_gemm / launch_bf16_gemm
 * (csrc/jit_kernels/fp8_gemm.hpp:11-151, fp8_dequant_gemm.hpp:24-95, bf16_gemm.hpp:16-78).
 *
 * A and B are K-major: A row i at a + i*lda, B row j at b + j*ldb (elements of the storage
 * type: bytes for e4m3 and packed e2m1, bf16 elements for DG_KIND_BF16).  D is row-major
 * with row stride ldd (elements of d_dtype).
 */
typedef struct dg_gemm_args {
    int32_t kind;                 /* DG_KIND_*                                               */
    int32_t gemm_type;            /* DG_GEMM_*                                               */
    const void *a, *b;
    void *d;
    const int16_t *sfa, *sfb;     /* required-layout SF; NULL for DG_KIND_BF16              */
    const void *bias;             /* [N] of d_dtype, or NULL                                 */
    const int32_t *grouped_layout;/* psum / m_indices / masked_m (see DG_GEMM_*)             */
    int32_t m, n, k;              /* logical sizes; for MASKED, m = rows per group           */
    int32_t num_groups;           /* batches / groups                                        */
    int64_t lda, ldb, ldd;
    int64_t batch_stride_a, batch_stride_b, batch_stride_d;   /* elements                   */
    int64_t sfa_ld, sfb_ld;       /* stride between k64 rows of SF (even, >= MN extent)      */
    int64_t sfa_batch_stride, sfb_batch_stride;
    int32_t d_dtype;              /* DG_DTYPE_*                                              */
    int32_t accumulate;           /* 1: D = D + alpha * A B^T                                */
    float alpha;                  /* 1.0f for plain                                          */
    int32_t alignment;            /* MGROUPED_* row alignment (128 or 256)                   */
    int32_t block_m, block_n;     /* 0 = library heuristic                                    */
    int32_t num_cus;              /* 0 = all CUs of the device (set_num_sms)                 */
    int32_t split_k;              /* K split: 0 = library heuristic, 1 = off, > 1 = forced   */
                                  /* (dense / batched GEMMs with a workspace only)           */
    void *workspace;              /* device scratch for split-K, or NULL (no split)          */
    int64_t workspace_bytes;      /* its size; see dg_gemm_workspace_size()                  */
    int32_t epilogue;             /* DG_EPI_*                                                */
    int16_t *sfd;                 /* DG_DTYPE_FP8_E4M3 only: output SF, int16 pairs of UE8M0 bytes;
                                     pair p = (batch * n + col) / 64 of row `row` at
                                     sfd[p * sfd_ld + row], lower byte = the even 32 columns      */
    int64_t sfd_ld;               /* >= m                                                    */
    int32_t jit;                  /* 1: launch a kernel compiled at run time for this problem
                                     (see dg_jit_compile); 0: the ahead-of-time tile menu       */
    int32_t compiled_dims;        /* jit only: DG_COMPILED_* sizes fixed at compile time (the
                                     reference's compiled_dims, csrc/jit_kernels/fp8_gemm.hpp:
                                     42-44); the GEMM type and K split always are              */
    int32_t library_workspace;    /* 1 (with workspace = NULL): a split-K plan takes its workspace
                                     from the library, one per (device, stream), allocated on first
                                     need, zero-filled, only ever grown and never freed (a captured
                                     graph may hold it).  Growing it while the stream is being
                                     captured is an error: run the call once before the capture. */
    int32_t a_mn_major;           /* 1: A is stored [K][M] (M contiguous; lda = stride between its K
                                     rows, in elements), read in place.  e4m3 x e4m3 and bf16 x bf16
                                     dense, batched and K-grouped GEMMs on the 256-row 128-byte-stage
                                     tiles only; any
                                     other plan fails with DG_ENOKERNEL (callers then copy to K-major).
                                     The reference's operand majors: deep_gemm/include/deep_gemm/
                                     fp8_gemm.hpp:18-35.                                            */
    int32_t b_mn_major;           /* 1: B is stored [K][N], likewise                                 */
} dg_gemm_args;

#define DG_COMPILED_M 1
#define DG_COMPILED_N 2
#define DG_COMPILED_K 4

/* Launch one GEMM.  Entry point replacing deep_gemm::launch_fp8_gemm /
 * launch_fp4_gemm / launch_fp8_dequant_gemm / launch_bf16_gemm (see dg_gemm_args). */
int dg_gemm(const dg_gemm_args *args, void *stream);

/* Runtime compilation (replaces the reference's deep-jit runtime, csrc/jit/jit.hpp:16-92, and
 * the compile-without-load of its dry-run mode, csrc/jit_kernels/fp8_gemm.hpp:75-78).
 * dg_jit_compile builds -- or finds in the DG_JIT_CACHE_DIR caches -- the kernel dg_gemm would
 * launch for `args` with jit = 1, without launching it (nothing touches the device).  Kernels are
 * compiled in-process with hipRTC for gfx950 from the headers in the include directory
 * (default: csrc/ next to the library's directory). */
int dg_jit_compile(const dg_gemm_args *args);
int dg_jit_set_include_dir(const char *dir);
/* Counters since load: hipRTC compilations, code objects read from the disk cache, launches of
 * an already loaded kernel. */
int dg_jit_stats(int64_t *compiled, int64_t *disk_hits, int64_t *memory_hits);

/*
 * Scale-factor layout transform.  Replaces launch_transform_sf
 * (csrc/jit_kernels/transform_sf.hpp:15-105) behind
 * transform_sf_into_required_layout (csrc/apis/layout.hpp:68-92).
 *
 * src: [num_batches][sf_mn][sf_k] of DG_SF_F32 (sf_k = ceil(K / gran_k)) or DG_SF_I16
 *      (sf_k = ceil(K / 64)), element (b, i, j) at src[b*stride_b + i*stride_mn + j*stride_k].
 * dst: packed int16, element (b, mn, k64) at dst[b*dst_stride_b + k64*ld + mn_idx] with
 *      ld = align(mn, 2), k64 < ceil(K/64), mn_idx < ld; mn_idx == mn (odd mn) is written 0.
 *      Row mn_idx < mn takes SF row mn_idx / gran_mn.  dst_stride_b >= ceil(K/64) * ld.
 * gran_k: 32 or 128 for DG_SF_F32 (128 repeats each exponent over four 32-blocks), 32 for I16.
 * psum (optional, device int32[num_groups]): M-grouped padding rows
 *      [ceil(psum[g]/gran_mn), align(psum[g], alignment)/gran_mn) (in SF rows) become 0.
 *      With num_groups = -1 it is instead the m_indices of the mn rows (gran_mn 1, one batch):
 *      rows with a negative index are padding and become 0.  Padding SF rows are not validated.
 * err_flag (optional, device int32): set to 1 when an fp32 SF has sign or mantissa bits
 *      (the reference traps on this, deep_gemm/include/deep_gemm/transform_sf.hpp:13-21);
 *      NULL: the library's sticky DG_ERR_SF_INVALID word is set instead (dg_take_errors).
 */
int dg_transform_sf(const void *src, int32_t src_kind, int64_t stride_b, int64_t stride_mn,
                    int64_t stride_k, int32_t num_batches, int32_t sf_mn, int32_t sf_k,
                    int32_t mn, int32_t k, int32_t gran_mn, int32_t gran_k,
                    const int32_t *psum, int32_t num_groups, int32_t alignment,
                    int16_t *dst, int64_t dst_stride_b, int32_t *err_flag, void *stream);

/*
 * Scale-factor layout transform of a K-grouped operand.  Replaces launch_transform_sf with
 * GemmType::KGroupedContiguousWithPsumLayout behind transform_k_grouped_sf_into_required_layout
 * (csrc/apis/layout.hpp:94-111).  One batch, same src / dst layout as dg_transform_sf.
 * psum (device int32[num_groups], required): K ranges of the groups; the SF of the K padding
 *      between groups, columns [ceil(psum[g]/w), align(psum[g], alignment)/w) with w = gran_k
 *      (DG_SF_F32) or 64 (DG_SF_I16), becomes 0 and is never validated.  alignment % 64 == 0.
 */
int dg_transform_k_grouped_sf(const void *src, int32_t src_kind, int64_t stride_mn, int64_t stride_k,
                              int32_t sf_mn, int32_t sf_k, int32_t mn, int32_t k, int32_t gran_mn,
                              int32_t gran_k, const int32_t *psum, int32_t num_groups, int32_t alignment,
                              int16_t *dst, int32_t *err_flag, void *stream);

/*
 * MN-major -> K-major operand copy.  The reference's kernels read MN-major operands in place
 * (its TMA / fractal loaders, deep_gemm/include/deep_gemm/ascend/copy.hpp); this build's GEMM
 * streams K-major rows, so an MN-major A / B (the tn / nn / tt layouts, K-grouped wgrad operands,
 * einsum views) is transposed once with this entry point before dg_gemm.
 * src element (b, k, mn) at src[b*src_batch_stride + k*src_ld + mn] (elements of elem_bytes = 1
 * or 2); dst element (b, mn, k) at dst[b*dst_batch_stride + mn*dst_ld + k] for k < k_padded,
 * zero for k >= k.  dst rows and batches 16-byte aligned.
 */
int dg_transpose_to_k_major(const void *src, int32_t elem_bytes, int32_t batches, int64_t src_batch_stride,
                            int64_t src_ld, int32_t k, int32_t mn, void *dst, int64_t dst_batch_stride,
                            int64_t dst_ld, int32_t k_padded, void *stream);

/*
 * FP4 (e2m1) operand packed along MN -> packed along K (the reference takes FP4 operands of either
 * major, deep_gemm/include/deep_gemm/fp8_gemm.hpp:18-35; this build's kernels read FP4 packed along K).
 * src byte (b, k, j) = MN 2j (low nibble) and 2j + 1 (high) of K row k, at
 * src[b*src_batch_stride + k*src_ld + j]; dst byte (b, mn, j) = K 2j (low) and 2j + 1 (high) of MN
 * row mn, at dst[b*dst_batch_stride + mn*dst_ld + j], zero for K >= k up to k_padded (even).  Strides
 * in bytes; dst rows and batches 16-byte aligned.
 */
int dg_fp4_to_k_major(const void *src, int32_t batches, int64_t src_batch_stride, int64_t src_ld, int32_t k,
                      int32_t mn, void *dst, int64_t dst_batch_stride, int64_t dst_ld, int32_t k_padded,
                      void *stream);

/* Number of compute units of `device` (the reference's get_num_sms, csrc/apis/runtime.hpp:13-19). */
int dg_device_num_cus(int32_t device);

/*
 * Workspace dg_gemm() can use for `args` (0 when its plan does not split K).  The workspace is
 * device memory that must be zero-filled before its first use; every dg_gemm() call leaves it
 * zero-filled again, so one workspace serves any number of calls issued in order on one stream
 * (calls in flight at the same time need separate workspaces).  With a smaller workspace, or
 * none, dg_gemm() runs an unsplit plan.  Has no counterpart in the reference, whose kernels do
 * not split K; callers that cannot provide scratch simply pass NULL.
 */
int dg_gemm_workspace_size(const dg_gemm_args *args, int64_t *bytes);

/* dg_gemm() that allocates nothing and takes no workspace: a split-K plan keeps its tile counters
 * and fp32 partials in a fixed device array of the library, 16 MiB + 64 KiB, held by every device
 * the library runs on until the process ends (args->workspace must be NULL and workspace_bytes 0;
 * a problem whose split-K plan needs more scratch is rejected with an error).  No counterpart in
 * the reference: it is for callers that cannot allocate -- code under HIP graph capture, serving
 * loops, harnesses that forbid hipMalloc.  Calls on one device share that array: calls that
 * overlap in time on one device (different streams) race; calls issued in order on one stream do
 * not (each launch leaves the counters zero for the next). */
int dg_gemm_noalloc(const dg_gemm_args *args, void *stream);

/* Sticky error words (no counterpart in the reference, which stops on a device-side assertion:
 * deep_gemm/include/deep_gemm/transform_sf.hpp:13-21).  Kernels that meet invalid input set a
 * word of host-mapped pinned memory instead of trapping; the host reads the words without any
 * stream synchronisation.
 *   DG_ERR_SF_INVALID  a float32 SF given to dg_transform_sf / dg_transform_k_grouped_sf (with
 *                      err_flag = NULL) had sign or mantissa bits set;
 *   DG_ERR_M_INDICES   an M-grouped m_indices layout (DG_GEMM_MGROUPED_IDX) was not padded to
 *                      `alignment`: some alignment-row block mixed two group ids, had a group id
 *                      after a padding row, or held an id >= num_groups.
 * dg_take_errors returns the DG_ERR_* bits set by kernels that completed since the last call and
 * clears them; after a hipStreamSynchronize (or event wait) it covers every call issued before
 * it, which is how a caller checks a given call at a sync point of its choosing.  dg_error_words returns the host address of the words (word i != 0: bit i). */
#define DG_ERR_SF_INVALID 1u
#define DG_ERR_M_INDICES 2u
/* The split-K workspace the library holds for (current device, stream) -- see library_workspace in
 * dg_gemm_args -- or NULL / 0 before a call needed one.  Nothing is allocated (inspection). */
int dg_stream_workspace(void *stream, void **ptr, int64_t *bytes);
uint32_t dg_take_errors(void);
const uint32_t *dg_error_words(void);

/* Tile shape dg_gemm() would pick for `args` (block_m, block_n written to the pointers). */
int dg_select_config(const dg_gemm_args *args, int32_t *block_m, int32_t *block_n);

/* The launch dg_gemm() would make for `args`, described without launching (nothing touches the
 * device).  Replaces the reference's GemmConfig / LaunchOptions as its heuristic returns them
 * (csrc/jit_kernels/gemm_config.hpp:39-95, csrc/jit_kernels/heuristics.hpp:92-98): the reference
 * launches `num_blocks = num_cores` persistent blocks; here `grid` is the workgroup count, equal
 * to min(tiles, num_cus) for a persistent launch (set_num_sms caps it) and to the tile count
 * (times split_k) otherwise. */
typedef struct dg_launch_info {
    int32_t block_m, block_n;     /* tile (skinny kernel: rows of A staged x strip columns)       */
    int64_t grid;                 /* workgroups launched                                          */
    int32_t threads;              /* threads per workgroup                                        */
    int64_t tiles;                /* output tiles (strips) of the problem                         */
    int32_t split_k;              /* K ranges per tile (1 = unsplit)                              */
    int32_t persistent;           /* 1: workgroups walk tiles (grid < tiles possible)             */
    int32_t skinny;               /* 1: the decode-shape kernel, 2: its shared-ring variant, 3: the decode GEMV kernel (block_m = M rows served, block_n = rows of B per workgroup, 64 / its K split) */
    int64_t plan_workgroups;      /* workgroups of the plan; under a CU cap (num_cus below the
                                     device's CUs) they go out in stream-ordered launches of at
                                     most `grid` <= num_cus workgroups each (the persistent kernel:
                                     one launch of `grid` workgroups walking every tile)          */
    int32_t split_reduce;         /* 1: a second launch sums the split-K partials (one wave per
                                     32x32 block of D) instead of each tile's last workgroup      */
} dg_launch_info;
int dg_launch_plan(const dg_gemm_args *args, dg_launch_info *info);

/* Message of the last failing call on this thread ("" if none). */
const char *dg_last_error(void);

/* Library version string. */
const char *dg_version(void);

#ifdef __cplusplus
}
#endif

#endif /* DEEP_GEMM_AMD_H_ */
