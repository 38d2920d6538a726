// Shared device/host helpers for the gfx950 flash-topk-attention kernels.
//
// Conventions used by every kernel in this library:
//  * One wavefront = 64 lanes.  MFMA tiles are v_mfma_f32_32x32x16_{bf16,f16}:
//      A operand (32 x 16): lane l holds row (l & 31), k = 8*(l >> 5) + e, e = 0..7
//      B operand (16 x 32): lane l holds col (l & 31), k = 8*(l >> 5) + e
//      C/D       (32 x 32): lane l holds col (l & 31), rows
//                           (i >> 2) * 8 + (l >> 5) * 4 + (i & 3), i = 0..15
//    Any permutation of k that is applied identically to A and B is harmless,
//    which the P.V and dS.K products use to consume C-layout registers directly.
//  * Attention operands are laid out so that both MFMA operands are contiguous
//    along the contraction dimension: row-major [token][d] for QK^T-type
//    products and transposed [d][token] copies ("T layout", padded token
//    coordinates) for products that contract over tokens.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

typedef __bf16 fta_bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 fta_f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 fta_bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 fta_f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

#define FTA_INF __builtin_inff()

enum { FTA_DTYPE_BF16 = 0, FTA_DTYPE_F16 = 1 };

// Element traits: 16-bit storage type is always uint16_t in memory.
template <int DT>
struct Elem;

template <>
struct Elem<FTA_DTYPE_BF16> {
    static __device__ __forceinline__ f32x16 mma(uint4 a, uint4 b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(fta_bf16x8, a),
                                                       __builtin_bit_cast(fta_bf16x8, b), c, 0, 0, 0);
    }
    static __device__ __forceinline__ uint32_t pack2(float lo, float hi) {
        fta_bf16x2 v = {(__bf16)lo, (__bf16)hi};
        return __builtin_bit_cast(uint32_t, v);
    }
    static __device__ __forceinline__ float to_f32(uint16_t x) {
        return __builtin_bit_cast(float, (uint32_t)x << 16);
    }
};

template <>
struct Elem<FTA_DTYPE_F16> {
    static __device__ __forceinline__ f32x16 mma(uint4 a, uint4 b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(fta_f16x8, a),
                                                      __builtin_bit_cast(fta_f16x8, b), c, 0, 0, 0);
    }
    static __device__ __forceinline__ uint32_t pack2(float lo, float hi) {
        fta_f16x2 v = {(_Float16)lo, (_Float16)hi};
        return __builtin_bit_cast(uint32_t, v);
    }
    static __device__ __forceinline__ float to_f32(uint16_t x) {
        return (float)__builtin_bit_cast(_Float16, x);
    }
};

__device__ __forceinline__ float fta_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float fta_log2(float x) { return __builtin_amdgcn_logf(x); }

// Value from lane (l ^ 32).
__device__ __forceinline__ float fta_xor32(float x) { return __shfl_xor(x, 32, 64); }

// Row of the 32x32 C layout held in accumulator register i of lane l.
__device__ __forceinline__ int c_row(int i, int lane) { return (i >> 2) * 8 + (lane >> 5) * 4 + (i & 3); }

// Workgroups are dispatched round-robin over the 8 XCDs of an MI355X; remap the
// hardware id so that each XCD walks one contiguous range of logical ids
// (neighbouring q-tiles of the same head share K/V in that XCD's L2).
__device__ __forceinline__ int fta_xcd_remap(int hw_id, int total) {
    constexpr int kXcd = 8;
    int per = total / kXcd;
    int full = per * kXcd;
    if (hw_id >= full) return hw_id;
    return (hw_id % kXcd) * per + hw_id / kXcd;
}

__device__ __forceinline__ uint4 fta_zero4() { return make_uint4(0u, 0u, 0u, 0u); }

// Status codes returned by every extern "C" entry point (see include/fta.h).
#define FTA_OK 0
#define FTA_ERR_ARG 1
#define FTA_ERR_UNSUPPORTED 2
#define FTA_ERR_HIP 3
