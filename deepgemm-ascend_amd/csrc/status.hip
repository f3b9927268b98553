// Sticky error words that kernels set and the host reads without a synchronisation, and the
// m_indices layout check of M-grouped GEMMs.
//
// The reference stops on a device-side assertion when a float32 scale factor carries sign or
// mantissa bits (deep_gemm/include/deep_gemm/transform_sf.hpp:13-21).  Here the kernel that meets
// such an input stores 1 into a word of host-mapped pinned memory; the host API reads (and clears)
// the words at its next call and raises there, so the check costs no stream synchronisation and
// no memcpy node inside a captured graph (the kernels write through a fixed host-mapped pointer).
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstring>
#include <mutex>

#include "../../include/deep_gemm_amd.h"

extern "C" __attribute__((visibility("hidden"))) int dg_set_error(const char* msg);

namespace dg {

// words[i] != 0: error i happened (DG_ERR_* bit i) since the last dg_take_errors()
constexpr int kNumStatusWords = 2;

namespace {
std::once_flag g_status_once;
uint32_t* g_status_host = nullptr;     // host view of the pinned words
std::atomic<uint32_t*> g_status_dev{nullptr};   // device view (same memory)

void status_alloc() {
    void* h = nullptr;
    if (hipHostMalloc(&h, 64, hipHostMallocMapped | hipHostMallocPortable | hipHostMallocCoherent) != hipSuccess ||
        h == nullptr) {
        (void)hipGetLastError();
        return;
    }
    void* d = nullptr;
    if (hipHostGetDevicePointer(&d, h, 0) != hipSuccess || d == nullptr) {
        (void)hipGetLastError();
        return;
    }
    std::memset(h, 0, 64);
    g_status_host = static_cast<uint32_t*>(h);
    g_status_dev.store(static_cast<uint32_t*>(d), std::memory_order_release);
}
}  // namespace

// Device address of the status words (allocated on the first call; nullptr if the pinned
// allocation failed, and then kernels skip the checks that report through it).
uint32_t* status_words() {
    std::call_once(g_status_once, status_alloc);
    return g_status_dev.load(std::memory_order_acquire);
}

// The same, without allocating: nullptr until some call has allocated the words.
uint32_t* status_words_if_ready() {
    return g_status_dev.load(std::memory_order_acquire);
}

// m_indices of an M-grouped contiguous GEMM: every `alignment`-row block must hold one group id
// (0 <= id < num_groups) on a prefix of its rows and padding (< 0) on the rest -- the layout the
// grouped kernel's per-tile group lookup relies on.  Thread r checks row r against row r - 1 (with
// `status`), and (with `blk_end`) a row r that ends its id's rows within its block records r + 1 as
// the block's valid end (the run table's input; for a checked layout one row per block does).
__global__ __launch_bounds__(256) void check_m_indices_kernel(const int32_t* idx, int m, int alignment,
                                                              int num_groups, uint32_t* status, int32_t* blk_end) {
    const int r = blockIdx.x * 256 + threadIdx.x;
    if (r >= m) return;
    const int v = idx[r];
    if (status != nullptr) {
        bool bad = v >= num_groups;
        if (v >= 0 && r % alignment != 0) bad = bad || idx[r - 1] != v;
        if (bad) status[1] = 1u;
    }
    if (blk_end != nullptr && v >= 0 && (r + 1 == m || (r + 1) % alignment == 0 || idx[r + 1] != v))
        blk_end[r / alignment] = r + 1;
}

int check_m_indices(const int32_t* idx, int m, int alignment, int num_groups, hipStream_t st, bool may_alloc,
                    int32_t* blk_end) {
    uint32_t* status = may_alloc ? status_words() : status_words_if_ready();
    if ((status == nullptr && blk_end == nullptr) || m <= 0) return DG_OK;
    hipLaunchKernelGGL(check_m_indices_kernel, dim3((unsigned)((m + 255) / 256)), dim3(256), 0, st, idx, m, alignment,
                       num_groups, status, blk_end);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        dg_set_error(hipGetErrorString(e));
        return DG_ELAUNCH;
    }
    return DG_OK;
}

// Runs of an m_indices layout: maximal sequences of `alignment`-row blocks whose first rows carry
// the same group id (-1: padding).  Output: runs[0] = the number of runs, then (first row, group,
// valid end) per run; a run ends where the next begins (the last at m), and its valid end is where the
// run's group ends in its final block (`blk_end`, from check_m_indices_kernel; the padding rows after it
// are neither loaded nor multiplied by the anchored tiles; rows before it keep their per-row id check).
// One workgroup: each thread takes a contiguous span of blocks, counts the runs starting there, and a
// workgroup prefix sum places them.
constexpr int kRunThreads = 1024;
__global__ __launch_bounds__(kRunThreads) void m_indices_runs_kernel(const int32_t* idx, int m, int alignment,
                                                                    int32_t* runs, const int32_t* blk_end) {
    __shared__ int counts[kRunThreads];
    const int tid = threadIdx.x;
    const int nblk = (m + alignment - 1) / alignment;
    const int per = (nblk + kRunThreads - 1) / kRunThreads;
    const int b0 = min(nblk, tid * per), b1 = min(nblk, b0 + per);
    int n = 0;
    for (int b = b0; b < b1; ++b)
        if (b == 0 || idx[(int64_t)b * alignment] != idx[(int64_t)(b - 1) * alignment]) ++n;
    counts[tid] = n;
    __syncthreads();
    for (int off = 1; off < kRunThreads; off <<= 1) {
        const int v = tid >= off ? counts[tid - off] : 0;
        __syncthreads();
        counts[tid] += v;
        __syncthreads();
    }
    int r = counts[tid] - n;   // runs before this thread's span
    for (int b = b0; b < b1; ++b) {
        const int g = idx[(int64_t)b * alignment];
        if (b == 0 || g != idx[(int64_t)(b - 1) * alignment]) {
            runs[1 + 3 * r] = b * alignment;
            runs[2 + 3 * r] = g;
            ++r;
        }
        // the run's final block (the next block starts another run, or there is none): its valid end
        if (b + 1 == nblk || idx[(int64_t)(b + 1) * alignment] != g) {
            const int lo = b * alignment + 1, hi = min(m, (b + 1) * alignment);
            int e = hi;
            if (g >= 0) {
                e = min(hi, max(lo, blk_end[b]));   // (clamped: an unchecked layout may leave any value)
            } else {
                while (e > lo && idx[e - 1] != g) --e;   // (padding runs: no block end recorded)
            }
            runs[3 * r] = e;   // (run r - 1, the one this block belongs to)
        }
    }
    if (tid == kRunThreads - 1) runs[0] = counts[tid];
}

int m_indices_runs(const int32_t* idx, int m, int alignment, int32_t* runs, const int32_t* blk_end, hipStream_t st) {
    hipLaunchKernelGGL(m_indices_runs_kernel, dim3(1), dim3(kRunThreads), 0, st, idx, m, alignment, runs, blk_end);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        dg_set_error(hipGetErrorString(e));
        return DG_ELAUNCH;
    }
    return DG_OK;
}

}  // namespace dg

extern "C" uint32_t dg_take_errors(void) {
    // (no allocation: before any call has allocated the words there is nothing to report)
    if (dg::status_words_if_ready() == nullptr) return 0;
    uint32_t bits = 0;
    for (int i = 0; i < dg::kNumStatusWords; ++i) {
        auto* w = reinterpret_cast<std::atomic<uint32_t>*>(dg::g_status_host + i);
        if (w->exchange(0u, std::memory_order_acq_rel) != 0u) bits |= 1u << i;
    }
    return bits;
}

extern "C" const uint32_t* dg_error_words(void) {
    dg::status_words();
    return dg::g_status_host;
}
