// Shared device/host definitions for the gfx950 block-scaled GEMM family.
#pragma once

// (The runtime compiler, hipRTC, brings its own HIP definitions and fixed-width types.)
#ifndef __HIPCC_RTC__
#include <hip/hip_runtime.h>
#include <stdint.h>
#else
using __hip_internal::int8_t;
using __hip_internal::uint8_t;
using __hip_internal::int16_t;
using __hip_internal::uint16_t;
using __hip_internal::int32_t;
using __hip_internal::uint32_t;
using __hip_internal::int64_t;
using __hip_internal::uint64_t;
#endif

namespace dg {

typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef int i32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) void lds_void;

// Operand format pair (A x B).  Values match DG_KIND_* in include/deep_gemm_amd.h.
enum Kind : int { kFP8FP8 = 0, kFP8FP4 = 1, kFP4FP4 = 2, kBF16 = 3 };
// Work decomposition.  Values match DG_GEMM_* in include/deep_gemm_amd.h.
enum GemmType : int { kNormal = 0, kBatched = 1, kMGroupedPsum = 2, kMGroupedIdx = 3, kMasked = 4, kKGrouped = 5 };

// MFMA operand-format codes of v_mfma_scale_f32_16x16x128_f8f6f4 (cbsz / blgp).
constexpr int kFmtE4M3 = 0;
constexpr int kFmtE2M1 = 4;

// Buffer-resource word 3 for raw (stride 0) loads with range checking on gfx9-class parts.
constexpr uint32_t kBufferRsrcWord3 = 0x00020000u;
// voffset that is always beyond num_records: such a lane reads zeros.
// Buffer-instruction cache-policy bit sc0: a load that misses the CU's L1 (served by the L2).
constexpr int kCacheSc0 = 1;
// Buffer-instruction cache-policy bit sc1 (device scope): a store is written through to memory
// and a load is served coherently for every XCD, so partials exchanged between workgroups on
// different XCDs (each XCD has its own L2) need no L2 writeback or invalidate.
constexpr int kCacheSc1 = 16;
constexpr uint32_t kOOBOffset = 0x80000000u;

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

// Two floats -> packed bf16 pair (low = a), round-to-nearest-even: v_cvt_pk_bf16_f32 on gfx950.
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
    const bf16x2 h = __builtin_convertvector(f32x2{a, b}, bf16x2);
    return __builtin_bit_cast(uint32_t, h);
}

__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
    return (uint16_t)(pack_bf16x2(f, 0.f) & 0xffffu);
}

__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
    return __builtin_bit_cast(float, ((uint32_t)h) << 16);
}

__host__ __device__ __forceinline__ int ceil_div(int a, int b) { return (a + b - 1) / b; }
__host__ __device__ __forceinline__ int64_t ceil_div64(int64_t a, int64_t b) { return (a + b - 1) / b; }
__host__ __device__ __forceinline__ int64_t align_up64(int64_t a, int64_t b) { return ceil_div64(a, b) * b; }
__host__ __device__ __forceinline__ int align_up(int a, int b) { return ceil_div(a, b) * b; }

}  // namespace dg
