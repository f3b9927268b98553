// Thin PyTorch extension: the common GEMM calls validated, their scale factors passed through (or
// transformed) and launched from C++, so a call costs a few microseconds of host time.
//
// It covers the reference's hot entry points (csrc/apis/gemm.hpp:225-256 fp8_fp4_gemm,
// :289-324 m_grouped_fp8_fp4_gemm_contiguous, :424-453 bf16_gemm, csrc/apis/layout.hpp:37-92
// for the scale-factor pass-through and transform) for K-major, 16-byte-aligned operands with no
// bias, alpha or output epilogue.  For anything else -- and for any input these checks would
// reject -- the entry returns false and the Python layer runs its general path, which raises the
// reference's error messages.  The library is reached through function pointers the Python layer
// hands over from the loaded libdeep_gemm_amd.so, so both layers always use the same library.
#include <torch/extension.h>

#include <cstdint>
#include <cstring>
#include <stdexcept>
#include <string>

#include "../../include/deep_gemm_amd.h"

namespace {

using GemmFn = int (*)(const dg_gemm_args*, void*);
using TransformFn = int (*)(const void*, int32_t, int64_t, int64_t, int64_t, int32_t, int32_t, int32_t, int32_t,
                            int32_t, int32_t, int32_t, const int32_t*, int32_t, int32_t, int16_t*, int64_t, int32_t*,
                            void*);
using TakeFn = uint32_t (*)();
using LastErrorFn = const char* (*)();

GemmFn g_gemm = nullptr;
TransformFn g_transform = nullptr;
TakeFn g_take = nullptr;
LastErrorFn g_last_error = nullptr;
const volatile uint32_t* g_words = nullptr;

constexpr int kFP8FP8 = 0, kFP8FP4 = 1, kFP4FP4 = 2, kBF16 = 3;
constexpr int kNormal = 0, kPsum = 2, kIdx = 3, kMasked = 4;

void init(int64_t gemm, int64_t transform, int64_t take, int64_t last_error, int64_t words) {
    g_gemm = reinterpret_cast<GemmFn>(gemm);
    g_transform = reinterpret_cast<TransformFn>(transform);
    g_take = reinterpret_cast<TakeFn>(take);
    g_last_error = reinterpret_cast<LastErrorFn>(last_error);
    g_words = reinterpret_cast<const volatile uint32_t*>(words);
}

void check_rc(int rc) {
    if (rc != 0) {
        const char* msg = g_last_error != nullptr ? g_last_error() : nullptr;
        throw std::runtime_error(msg != nullptr && msg[0] ? msg : ("deep_gemm error " + std::to_string(rc)));
    }
}

// Errors that kernels of earlier calls reported through the library's sticky words (read with no
// synchronisation; the words live in host-mapped memory).
uint32_t pending_errors() {
    if (g_words == nullptr || (g_words[0] == 0u && g_words[1] == 0u)) return 0;
    return g_take();
}

// The same words as the Python layer's message (deep_gemm/_lib.py, error_message).
std::string error_message(uint32_t bits) {
    std::string msg;
    if (bits & DG_ERR_SF_INVALID)
        msg += "Invalid float32 SF: only the 8-bit exponent may be set (sign and mantissa must be 0)";
    if (bits & DG_ERR_M_INDICES) {
        if (!msg.empty()) msg += "; ";
        msg += "m_indices is not padded to the M-grouped alignment (every alignment-row block must hold one group "
               "id < num_groups followed only by -1 padding)";
    }
    return msg + " [reported by a kernel of an earlier deep_gemm call]";
}

int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }
int64_t align_up(int64_t a, int64_t b) { return ceil_div(a, b) * b; }

bool is_fp4(const at::Tensor& t) { return t.scalar_type() == at::kChar; }

// K-major check of the reference's get_major_type_ab (csrc/utils/layout.hpp:37-47), without its
// error (an ambiguous or MN-major operand goes to the general path).
bool k_major(const at::Tensor& t) {
    if (t.stride(-1) != 1) return false;
    return !(t.stride(-2) == 1 && t.size(-1) > 1 && t.size(-2) > 1);
}

// The kernel reads the operand in place: K rows of whole 16-byte units at 16-byte aligned
// addresses (the general path pads or transposes otherwise).
bool kernel_ready(const at::Tensor& t) {
    const int64_t elem = t.element_size();
    if ((t.size(-1) * elem) % 16 || (t.stride(-2) * elem) % 16 || (reinterpret_cast<uintptr_t>(t.data_ptr()) & 15))
        return false;
    if (t.dim() == 3 && (t.stride(0) * elem) % 16) return false;
    return true;
}

// Scale factors in the kernels' layout: `sf` itself when it already is (check_sf_layout,
// csrc/apis/layout.hpp:37-65), else the output of the transform kernel
// (csrc/jit_kernels/transform_sf.hpp:15-105).  An undefined tensor: the general path decides.
// psum: the M-grouped layout of A's rows (its m_indices when rows_by_index), whose padding rows
// are skipped.
at::Tensor kernel_sf(const at::Tensor& sf, int64_t mn, int64_t k, int64_t gran_mn, int64_t gran_k, int64_t groups,
                     const at::Tensor* psum, bool rows_by_index, int64_t alignment, int64_t stream) {
    const auto dt = sf.scalar_type();
    if (dt != at::kFloat && dt != at::kShort) return {};
    const int64_t rank = groups > 0 ? 3 : 2;
    if (sf.dim() != rank || !(sf.stride(-1) == 1 || sf.stride(-2) == 1)) return {};
    if (groups > 0 && sf.size(0) != groups) return {};
    int64_t div_k = 64;
    if (dt == at::kFloat) {
        if (gran_k != 32 && gran_k != 128) return {};
        div_k = gran_k;
    } else if (gran_k != 32) {
        return {};
    }
    if (sf.size(-2) != ceil_div(mn, gran_mn) || sf.size(-1) != ceil_div(k, div_k)) return {};
    if (dt == at::kShort && gran_mn == 1 && sf.stride(-2) == 1 && sf.stride(-1) == align_up(sf.size(-2), 2)) {
        if (groups == 0 || sf.stride(0) == sf.stride(-1) * sf.size(-1)) return sf;
    }
    if (gran_mn < 1 || gran_mn > 128 || (gran_mn & (gran_mn - 1)) || !sf.is_cuda()) return {};
    if (rows_by_index && (gran_mn != 1 || groups > 0)) psum = nullptr;
    const int64_t nb = groups > 0 ? groups : 1;
    const int64_t k64 = ceil_div(k, 64), ld = align_up(mn, 2);
    at::Tensor out = at::empty({nb, k64, ld}, sf.options().dtype(at::kShort));
    const int64_t sb = groups > 0 ? sf.stride(0) : 0;
    check_rc(g_transform(sf.data_ptr(), dt == at::kFloat ? DG_SF_F32 : DG_SF_I16, sb, sf.stride(-2), sf.stride(-1),
                         (int32_t)nb, (int32_t)sf.size(-2), (int32_t)sf.size(-1), (int32_t)mn, (int32_t)k,
                         (int32_t)gran_mn, (int32_t)gran_k,
                         psum != nullptr ? psum->data_ptr<int32_t>() : nullptr,
                         psum == nullptr ? 0 : rows_by_index ? -1 : (int32_t)psum->numel(), (int32_t)alignment,
                         out.data_ptr<int16_t>(), k64 * ld, nullptr, reinterpret_cast<void*>(stream)));
    out = out.slice(2, 0, mn).transpose(-2, -1);
    return groups > 0 ? out : out.squeeze(0);
}

int operand_kind(const at::Tensor& a, const at::Tensor& b) {
    const auto ta = a.scalar_type(), tb = b.scalar_type();
    if (ta == at::kFloat8_e4m3fn && tb == at::kFloat8_e4m3fn) return kFP8FP8;
    if (ta == at::kFloat8_e4m3fn && tb == at::kChar) return kFP8FP4;
    if (ta == at::kChar && tb == at::kChar) return kFP4FP4;
    if (ta == at::kBFloat16 && tb == at::kBFloat16) return kBF16;
    return -1;
}

// GEMM over K-major operands:
//   gemm_type 0 (dense): a [M, K], b [N, K], d [M, N], c = None or d itself (accumulate);
//   gemm_type 2 / 3 (M-grouped contiguous, psum / m_indices): b [G, N, K], layout int32;
//   gemm_type 4 (masked): a [G, M, K], b [G, N, K], d [G, M, N], layout = masked_m.
// recipes: (gran_a_mn, gran_a_k, gran_b_mn, gran_b_k); num_cus 0 = the device's CUs.
bool gemm(int64_t gemm_type, const at::Tensor& a, const c10::optional<at::Tensor>& sfa_in, const at::Tensor& b,
          const c10::optional<at::Tensor>& sfb_in, const at::Tensor& d, const c10::optional<at::Tensor>& c,
          const c10::optional<at::Tensor>& layout, int64_t gran_a_mn, int64_t gran_a_k, int64_t gran_b_mn,
          int64_t gran_b_k, int64_t num_cus, int64_t alignment, int64_t stream) {
    if (g_gemm == nullptr) return false;
    if (const uint32_t bits = pending_errors()) throw std::runtime_error(error_message(bits));
    const int kind = operand_kind(a, b);
    if (kind < 0) return false;
    const bool bf16 = kind == kBF16;
    const bool grouped = gemm_type == kPsum || gemm_type == kIdx;
    const bool masked = gemm_type == kMasked;
    if (!(gemm_type == kNormal || grouped || masked)) return false;
    const int64_t ra = masked ? 3 : 2, rb = gemm_type == kNormal ? 2 : 3;
    if (a.dim() != ra || b.dim() != rb || d.dim() != ra) return false;
    if (!k_major(a) || !k_major(b) || d.stride(-1) != 1) return false;
    const auto dt = d.scalar_type();
    if (dt != at::kBFloat16 && dt != at::kFloat) return false;
    if (!a.is_cuda() || a.device() != d.device() || b.device() != d.device()) return false;
    const int64_t k = a.size(-1) * (is_fp4(a) ? 2 : 1);
    const int64_t kb = b.size(-1) * (is_fp4(b) ? 2 : 1);
    const int64_t m = a.size(-2), n = b.size(-2);
    if (k != kb || m == 0 || n == 0 || k == 0) return false;
    if (d.size(-2) != m || d.size(-1) != n) return false;
    const int64_t groups = rb == 3 ? b.size(0) : 1;
    if (masked && (a.size(0) != groups || d.size(0) != groups)) return false;
    if (!kernel_ready(a) || !kernel_ready(b)) return false;
    bool accumulate = false;
    if (c.has_value()) {
        const at::Tensor& ct = *c;
        if (gemm_type != kNormal || ct.data_ptr() != d.data_ptr() || ct.sizes() != d.sizes() ||
            ct.strides() != d.strides() || ct.scalar_type() != dt)
            return false;
        accumulate = true;
    }
    const at::Tensor* lay = nullptr;
    if (gemm_type != kNormal) {
        if (!layout.has_value()) return false;
        lay = &*layout;
        if (lay->scalar_type() != at::kInt || !lay->is_contiguous() || lay->device() != d.device()) return false;
        const int64_t want = gemm_type == kIdx ? m : groups;
        if (lay->numel() != want) return false;
    }

    dg_gemm_args args;
    std::memset(&args, 0, sizeof(args));
    at::Tensor sfa_t, sfb_t;
    if (!bf16) {
        if (!sfa_in.has_value() || !sfb_in.has_value()) return false;
        // (validate both before launching either transform)
        const at::Tensor& sfa = *sfa_in;
        const at::Tensor& sfb = *sfb_in;
        if (sfa.device() != d.device() || sfb.device() != d.device()) return false;
        const at::Tensor* rows = grouped ? lay : nullptr;
        sfa_t = kernel_sf(sfa, m, k, gran_a_mn, gran_a_k, masked ? groups : 0, rows, gemm_type == kIdx, alignment,
                          stream);
        if (!sfa_t.defined()) return false;
        sfb_t = kernel_sf(sfb, n, k, gran_b_mn, gran_b_k, rb == 3 ? groups : 0, nullptr, false, alignment, stream);
        if (!sfb_t.defined()) return false;
        args.sfa = static_cast<const int16_t*>(sfa_t.data_ptr());
        args.sfb = static_cast<const int16_t*>(sfb_t.data_ptr());
        args.sfa_ld = sfa_t.stride(-1);
        args.sfb_ld = sfb_t.stride(-1);
        if (masked) args.sfa_batch_stride = sfa_t.stride(0);
        if (rb == 3) args.sfb_batch_stride = sfb_t.stride(0);
    }
    args.kind = kind;
    args.gemm_type = (int32_t)gemm_type;
    args.a = a.data_ptr();
    args.b = b.data_ptr();
    args.d = d.data_ptr();
    args.grouped_layout = lay != nullptr ? lay->data_ptr<int32_t>() : nullptr;
    args.m = (int32_t)m;
    args.n = (int32_t)n;
    args.k = (int32_t)k;
    args.num_groups = (int32_t)groups;
    args.lda = a.stride(-2);
    args.ldb = b.stride(-2);
    args.ldd = d.stride(-2);
    if (masked) {
        args.batch_stride_a = a.stride(0);
        args.batch_stride_d = d.stride(0);
    }
    if (rb == 3) args.batch_stride_b = b.stride(0);
    args.d_dtype = dt == at::kFloat ? DG_DTYPE_F32 : DG_DTYPE_BF16;
    args.accumulate = accumulate ? 1 : 0;
    args.alpha = 1.0f;
    args.alignment = (int32_t)alignment;
    args.num_cus = (int32_t)num_cus;
    args.library_workspace = gemm_type == kNormal ? 1 : 0;
    check_rc(g_gemm(&args, reinterpret_cast<void*>(stream)));
    return true;
}

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
    m.doc() = "deep_gemm C++ host path (validation, scale-factor pass-through and launch)";
    m.def("init", &init, "hand over the library's entry points");
    m.def("gemm", &gemm, "validate and launch one GEMM; false: the general path must handle the call");
}
