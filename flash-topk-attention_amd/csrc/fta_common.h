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
//  * Token tiles are staged row-major ([token][d]) in LDS.  QK^T-type products
//    read them with plain 16-byte LDS loads; products that contract over tokens
//    read the same tiles transposed with fta_tr_frag (ds_read_b64_tr_b16).
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

// gfx950 v_permlane32_swap on two registers (measured): afterwards
//   a = [a_lo | b_lo], b = [a_hi | b_hi]   (lo = lanes 0..31, hi = lanes 32..63)
// so for lane l, a + b = a_in[l] + a_in[l + 32] (l < 32) or b_in[l - 32] + b_in[l]
// (l >= 32).  Issued through asm (the compiler builtin gave wrong results with
// this toolchain); the s_nops keep it clear of VALU read/write hazards.
__device__ __forceinline__ void fta_swap32(float& a, float& b) {
    asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
}

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

// MFMA operand (A or B format) whose k index runs down the ROWS of a row-major
// LDS tile, read with the gfx950 LDS transpose load ds_read_b64_tr_b16:
//   element e of lane l = tile[(k0 + kperm(l, e)) * row + n0 + (l & 31)],
//   kperm(l, e) = 8 * (e >> 2) + 4 * (l >> 5) + (e & 3)
// (the same k permutation as the rows of the 32x32 C layout, so C-layout
// registers can be contracted against it directly).
// ds_read_b64_tr_b16 semantics (per 16-lane group, measured on gfx950): lane j
// receives element (j & 3) of the 64-bit words addressed by lanes
// 4e + (j >> 2), e = 0..3.  Lane i of a group therefore addresses row
// (i >> 2) and columns 4 * (i & 3) .. +3 of a 4 x 16 sub-block.
typedef short fta_s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) fta_s16x4 fta_lds_s16x4;
__device__ __forceinline__ uint4 fta_tr_frag(const uint16_t* tile, int row, int k0, int n0, int lane) {
    const int g = lane >> 4, i = lane & 15;
    const int r = k0 + 4 * (g >> 1) + (i >> 2);
    const int col = n0 + 16 * (g & 1) + 4 * (i & 3);
    const uint16_t* p0 = tile + r * row + col;
    const uint16_t* p1 = p0 + 8 * row;
    const fta_s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (fta_lds_s16x4*)(__attribute__((address_space(3))) uint16_t*)p0);
    const fta_s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (fta_lds_s16x4*)(__attribute__((address_space(3))) uint16_t*)p1);
    const uint2 l2 = __builtin_bit_cast(uint2, lo), h2 = __builtin_bit_cast(uint2, hi);
    return make_uint4(l2.x, l2.y, h2.x, h2.y);
}

// ---------------------------------------------------------------------------
// Swizzled token tiles filled by LDS DMA.
// gfx950 global_load_lds_dwordx4 writes 16 bytes per lane straight into LDS at
// M0 + 16 * lane (wave-uniform base, per-lane global address; measured on
// gfx950), so a wave instruction fills 1 KB of contiguous LDS and rows cannot
// be padded.  Rows of QSEG 16-byte slots are stored unpadded with slot j of
// row r at position j ^ x(r); the loading lane picks its global source from its
// physical position, the reading lane swizzles its address.
// x(r) is chosen from measured gfx950 LDS bank behaviour (64 banks of 4 bytes,
// SQ_LDS_BANK_CONFLICT):
//  * 16-byte reads (MFMA operand rows, lane = row) are served 16 lanes at a
//    time over 256 bytes: 16 consecutive rows reading one logical slot need
//    16 distinct bank positions, i.e. x bijective on r & 15 for rows of 256
//    bytes or more (an x built from r & 7 alone left rows r and r + 8 on the
//    same banks: a 2-way conflict on every operand read, 6.8e8 conflict cycles
//    per C3-iid sparse forward, 5.5e8 per C3 scoring launch);
//  * ds_read_b64_tr_b16 is served 32 lanes at a time over 256 bytes: 4
//    consecutive rows x 64 bytes, so bits 2..3 of x must differ across them.
// x(r) = (r & 3) << 2 | (r >> 2) & 3 meets both for 16 or more slots per row
// (V = 1 keeps the earlier 8-row form, which one kernel measured faster with);
// 8 slots (128-byte rows, two rows per bank line) use the row-pair form; 4
// slots need none.  12 and 20 slots use r & 3 (not tuned).
// ---------------------------------------------------------------------------
template <int QSEG, int V = 0>
struct FtaSwz {
    static_assert(QSEG % 4 == 0, "rows must be a multiple of 4 slots");
    __device__ static __forceinline__ int x(int r) {
        if constexpr (QSEG % 16 == 0 && V == 1) {
            return ((r & 1) << 2) | (((r >> 1) & 1) * 10) | ((r >> 2) & 1);
        } else if constexpr (QSEG % 16 == 0) {
            return ((r & 3) << 2) | ((r >> 2) & 3);
        } else if constexpr (QSEG == 8) {
            const int h = (r >> 1) & 7;
            return ((h & 1) << 2) | (h >> 1);
        } else if constexpr (QSEG == 4) {
            return 0;
        } else {
            return r & 3;
        }
    }
    // uint16 offset of logical slot j of row r
    __device__ static __forceinline__ int off(int r, int j) { return r * QSEG * 8 + ((j ^ x(r)) << 3); }
    // logical slot held at physical position p of row r
    __device__ static __forceinline__ int slot(int r, int p) { return p ^ x(r); }
};

// fta_tr_frag over a swizzled tile of QSEG slots per row.
template <int QSEG, int V = 0>
__device__ __forceinline__ uint4 fta_tr_frag_sw(const uint16_t* tile, int k0, int n0, int lane) {
    const int g = lane >> 4, i = lane & 15;
    const int r = k0 + 4 * (g >> 1) + (i >> 2);
    const int col = n0 + 16 * (g & 1) + 4 * (i & 3);
    const uint16_t* p0 = tile + FtaSwz<QSEG, V>::off(r, col >> 3) + (col & 7);
    const uint16_t* p1 = tile + FtaSwz<QSEG, V>::off(r + 8, col >> 3) + (col & 7);
    const fta_s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (fta_lds_s16x4*)(__attribute__((address_space(3))) uint16_t*)p0);
    const fta_s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (fta_lds_s16x4*)(__attribute__((address_space(3))) uint16_t*)p1);
    const uint2 l2 = __builtin_bit_cast(uint2, lo), h2 = __builtin_bit_cast(uint2, hi);
    return make_uint4(l2.x, l2.y, h2.x, h2.y);
}

// One wave-wide LDS DMA: lane l copies 16 (or 4) bytes from g to lds + 16 * l
// (or 4 * l).  `lds` must be wave-uniform.  Completion is tracked by vmcnt and
// waited for explicitly (fta_wait_vmcnt + barrier).  Issued through inline asm
// so the compiler's wait insertion does not see an LDS write in flight: with
// the builtin it waits for every outstanding DMA (vmcnt(0)) before each LDS
// read, which serialises a multi-stage pipeline.  Loads the compiler does track
// stay correct: DMAs unknown to it only make its own vmcnt waits stricter.
// An SALU write of M0 needs one wait state before an LDS DMA reads it (the
// compiler inserts it for its own code, not inside asm): hence the s_nop.
__device__ __forceinline__ uint32_t fta_lds_addr(const void* lds) {
    return __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)lds);
}
__device__ __forceinline__ void fta_dma16_at(const void* g, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g),
                 "s"(__builtin_amdgcn_readfirstlane(lds)) : "memory", "m0");
}
// The same DMA with a wave-uniform base (SGPR pair) and a 32-bit per-lane byte offset:
// one VGPR per address instead of two.
__device__ __forceinline__ void fta_dma16_so(const void* base, uint32_t voff, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(base),
                 "s"(__builtin_amdgcn_readfirstlane(lds)) : "memory", "m0");
}
__device__ __forceinline__ void fta_dma4_at(const void* g, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off" ::"v"(g),
                 "s"(__builtin_amdgcn_readfirstlane(lds)) : "memory", "m0");
}
__device__ __forceinline__ void fta_dma16(const void* g, void* lds) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(fta_lds_addr(lds)) : "memory", "m0");
}
__device__ __forceinline__ void fta_dma4(const void* g, void* lds) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off" ::"v"(g), "s"(fta_lds_addr(lds)) : "memory", "m0");
}

// s_waitcnt vmcnt(N) alone (expcnt and lgkmcnt left at their maxima).
template <int N>
__device__ __forceinline__ void fta_wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Status codes (FTA_OK / FTA_ERR_*) and FTA_NOALLOC_SCRATCH_BYTES come from the
// public header, so the library and its callers share one definition.
#include "fta.h"
