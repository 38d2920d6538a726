// Block-sparse attention forward and backward for gfx950.
//
// Reference semantics: flash_topk_attn_v2/sparse_attn.py:24-127 (forward),
// sparse_attn_bwd.py:111-294 (dQ, dK, dV), kernels
// csrc/sparse_attn_kernel.cu:6-365, csrc/sparse_attn_bwd_dq_kernel.cu:6-419,
// csrc/sparse_attn_bwd_dkv_kernel.cu:6-435.
//
// Design (MI355X-first, not a translation of the CuTe kernels):
//  * A workgroup owns 32-query tiles of one (b, h) (forward / dQ) or 32-key tiles
//    (dK/dV).  It builds, in LDS, a per-tile 32-bit column mask for every KV
//    block (resp. 32-query chunk) from the merged lists, takes the union of
//    the blocks any of its tiles needs, and stages each union block in LDS
//    once for all its tiles.  Tiles whose mask is empty skip the MFMAs; tiles
//    whose mask is partial mask columns.  This handles any q_block_size,
//    kv_block_size and virtual padding with one code path, and reuses every
//    gathered KV byte across up to 8 q-blocks.
//  * dK/dV walk the transposed membership (KV block -> q-blocks) directly, so no
//    atomics are needed on the gradient path.
//  * Operands that are contracted over tokens (V in P.V, K in dS.K, Q and dO in
//    the dK/dV products) are read from the same row-major LDS tiles with the
//    gfx950 LDS transpose load (fta_tr_frag), so each token tile is gathered
//    from HBM once and no transposed copies exist.
#include "fta_common.h"
#include "fta_host.h"

#include <algorithm>
#include <mutex>
#include <type_traits>

namespace fta {
int launch_sel_bitmap(const int32_t* merged, int BH, int QM, int W, int M, uint32_t* sel, hipStream_t st);
int launch_kv_order(const uint32_t* sel, int B, int H, int Hk, int M, int QW, int32_t* order, int32_t* head_work,
                    int32_t* head_perm, hipStream_t st);
int launch_head_order_merged(const int32_t* merged, int BH, int QM, int W, int M, int qpg, int32_t* head_work,
                             int32_t* head_perm, hipStream_t st);
}  // namespace fta

constexpr int kSeg = 512;    // KV blocks per mask segment (forward / dQ)
constexpr int kSegC = 1024;  // 32-query chunks per mask segment (dK/dV): N <= 32768 in one pass
constexpr int kBitsW = 64;   // bitmap words per KV block staged in LDS by dK/dV (QM <= 2048)

struct AttnArgs {
    const uint16_t* q;
    int64_t q_sb, q_sh, q_sn;
    const uint16_t* k;
    int64_t k_sb, k_sh, k_sn;
    const uint16_t* v;
    int64_t v_sb, v_sh, v_sn;
    const uint16_t* dout;
    int64_t d_sb, d_sh, d_sn;
    const int32_t* merged;  // [BH][QM][W]
    const uint32_t* sel;    // [BH][Mkv][QW] membership bitmap (dK/dV)
    const int32_t* kv_order;  // [B*Hk][Mkv] dK/dV launch order of the KV blocks (null: natural order)
    const int32_t* head_perm;  // [B*Hk] (dK/dV) or [B*H] (forward, dQ): head at each head position (null: natural order)
    int QM, W, QW;
    uint16_t* out0;  // o (forward) / dq / dk
    int64_t o0_sb, o0_sh, o0_sn;
    uint16_t* out1;  // dv
    int64_t o1_sb, o1_sh, o1_sn;
    float* lse;             // forward output, natural log, [BH][N]
    const float* lse_in;    // backward input
    const float* lse2_in;   // lse_in * log2(e), [BH][N] (workspace; dK/dV split kernel)
    const float* delta_in;  // backward input
    int H, N, Dreal, g, kvb, q_pad, kv_pad, Mkv, NC;
    int Hk, G;  // K/V heads and query heads per K/V head (G = H / Hk; 1 without GQA)
    float c, scale;
    int wg_per_bh, total;
    // forward split over the union walk (nsplit > 1, small grids): partial
    // unnormalised O [nsplit][nbh][npq][Dk] and (m, L) [nsplit][nbh][npq], by
    // padded query position, merged by fta_fwd_combine_kernel
    int nsplit, nbh, npq;
    float* part_o;
    float2* part_ml;
};

// Bits [lo, hi) of a 32-bit mask; lo and hi may lie anywhere (they are clamped
// to [0, 32] first, so a range wholly outside the word gives 0).
__device__ __forceinline__ uint32_t fta_range_bits(int lo, int hi) {
    lo = max(lo, 0);
    hi = min(hi, 32);
    if (hi <= lo) return 0u;
    const uint32_t up = (hi == 32) ? 0xffffffffu : ((1u << hi) - 1u);
    const uint32_t dn = (1u << lo) - 1u;
    return up & ~dn;
}

// Column masks of the WG's query tiles for KV blocks [seg0, seg0 + segn), then
// the ascending union list.  Returns the list length.
template <int T>
__device__ int fta_build_q_masks(const AttnArgs& a, int bh, int p0, int seg0, int segn, uint32_t (*sMask)[kSeg],
                                 int* sList, int* s_tmp) {
    const int tid = threadIdx.x;
    for (int i = tid; i < T * kSeg; i += blockDim.x) sMask[i / kSeg][i % kSeg] = 0u;
    __syncthreads();
    const int pend = p0 + 32 * T;
    const int qb_lo = p0 / a.g;
    int qb_hi = (pend - 1) / a.g;
    if (qb_hi > a.QM - 1) qb_hi = a.QM - 1;
    const int vlo = a.q_pad, vhi = a.q_pad + a.N;  // valid padded query positions
    const int npairs = (qb_hi - qb_lo + 1) * a.W;
    for (int pi = tid; pi < npairs; pi += blockDim.x) {
        const int qb = qb_lo + pi / a.W;
        const int s = pi - (pi / a.W) * a.W;
        const int m = a.merged[((int64_t)bh * a.QM + qb) * a.W + s];
        if (m < seg0 || m >= seg0 + segn || m >= a.Mkv) continue;
        int lo = qb * a.g, hi = qb * a.g + a.g;
        lo = max(lo, max(p0, vlo));
        hi = min(hi, min(pend, vhi));
        if (lo >= hi) continue;
        for (int tau = (lo - p0) >> 5; tau <= (hi - 1 - p0) >> 5; ++tau) {
            const int tb = p0 + 32 * tau;
            const uint32_t bits = fta_range_bits(max(lo, tb) - tb, min(hi, tb + 32) - tb);
            atomicOr(&sMask[tau][m - seg0], bits);
        }
    }
    __syncthreads();
    int U = 0;
    for (int base = 0; base < segn; base += blockDim.x) {
        const int ml = base + tid;
        int any = 0;
        if (ml < segn) {
#pragma unroll
            for (int t = 0; t < T; ++t) any |= (sMask[t][ml] != 0u);
        }
        // block-wide exclusive scan of `any`
        const int lane = tid & 63, wave = tid >> 6;
        int x = any;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const int y = __shfl_up(x, off, 64);
            if (lane >= off) x += y;
        }
        if (lane == 63 && wave < 8) s_tmp[wave] = x;
        __syncthreads();
        const int nw = blockDim.x >> 6;
        int wbase = 0, tot = 0;
        for (int w = 0; w < nw; ++w) {
            const int t = s_tmp[w];
            if (w < wave) wbase += t;
            tot += t;
        }
        if (any) sList[U + wbase + x - any] = ml;
        __syncthreads();
        U += tot;
    }
    return U;
}

// ----------------------------------------------------------------------------
// Forward.  WG = 4 waves x TPW tiles x 32 queries.  For every union KV block,
// 64-key chunks of K and V (row layout) are double-buffered in LDS; V^T operands
// come from LDS transpose reads.
// Per tile: S^T = K Q^T (32 keys x 32 queries per MFMA), online softmax with a
// lazily rescaled running max (rescale only when the max grows by > 2^8),
// O^T += V^T P^T.
// ----------------------------------------------------------------------------
template <int DT, int D, int TPW, int NW>
__global__ __launch_bounds__(NW * 64, 1) void fta_sparse_fwd_kernel(AttnArgs a) {
    using E = Elem<DT>;
    constexpr int NTHR = NW * 64;
    constexpr int T = NW * TPW;
    constexpr int KS = D / 16;
    constexpr int DT32 = D / 32;
    constexpr int KROW = D + 8;
    constexpr int KSEG = D / 8;
    constexpr int KLOADS = (64 * KSEG + NTHR - 1) / NTHR;
    __shared__ __align__(16) uint16_t sK[2][64 * KROW];
    __shared__ __align__(16) uint16_t sV[2][64 * KROW];
    __shared__ uint32_t sMask[T][kSeg];
    __shared__ int sList[kSeg];
    __shared__ int s_tmp[8];

    const int wgi = fta_xcd_remap(blockIdx.x, a.total);
    const int bh = wgi / a.wg_per_bh;
    const int wq = wgi - bh * a.wg_per_bh;
    const int b = bh / a.H, h = bh - (bh / a.H) * a.H;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int hf = lane >> 5;
    const int p0 = wq * 32 * T;

    const uint16_t* qp = a.q + b * a.q_sb + h * a.q_sh;
    const uint16_t* kp = a.k + b * a.k_sb + (h / a.G) * a.k_sh;
    const uint16_t* vp = a.v + b * a.v_sb + (h / a.G) * a.v_sh;

    uint4 qf[TPW][KS];
#pragma unroll
    for (int tt = 0; tt < TPW; ++tt) {
        const int t = p0 + 32 * (wave * TPW + tt) + (lane & 31) - a.q_pad;
        const bool ok = t >= 0 && t < a.N;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            const int d = ks * 16 + hf * 8;
            qf[tt][ks] = (ok && d < a.Dreal) ? *reinterpret_cast<const uint4*>(qp + (int64_t)t * a.q_sn + d)
                                             : fta_zero4();
        }
    }

    f32x16 oacc[TPW][DT32];
#pragma unroll
    for (int tt = 0; tt < TPW; ++tt)
#pragma unroll
        for (int dt = 0; dt < DT32; ++dt)
#pragma unroll
            for (int i = 0; i < 16; ++i) oacc[tt][dt][i] = 0.f;
    float m_run[TPW], l_run[TPW];
#pragma unroll
    for (int tt = 0; tt < TPW; ++tt) {
        m_run[tt] = -FTA_INF;
        l_run[tt] = 0.f;
    }

    const int nch = (a.kvb + 63) >> 6;
    uint4 kst[KLOADS], vst[KLOADS];

    for (int seg0 = 0; seg0 < a.Mkv; seg0 += kSeg) {
        const int segn = min(kSeg, a.Mkv - seg0);
        const int U = fta_build_q_masks<T>(a, bh, p0, seg0, segn, sMask, sList, s_tmp);
        if (U == 0) continue;
        const int iters = U * nch;

        auto load = [&](int it) {
            const int u = it / nch, ch = it - (it / nch) * nch;
            const int m = seg0 + sList[u];
            const int kb = m * a.kvb - a.kv_pad + ch * 64;
            const int rem = a.kvb - ch * 64;
#pragma unroll
            for (int i = 0; i < KLOADS; ++i) {
                const int s = tid + i * NTHR;
                const int row = s / KSEG, sg = s - (s / KSEG) * KSEG;
                const int t = kb + row;
                const bool ok = s < 64 * KSEG && row < rem && t >= 0 && t < a.N && sg * 8 < a.Dreal;
                kst[i] = ok ? *reinterpret_cast<const uint4*>(kp + (int64_t)t * a.k_sn + sg * 8) : fta_zero4();
                vst[i] = ok ? *reinterpret_cast<const uint4*>(vp + (int64_t)t * a.v_sn + sg * 8) : fta_zero4();
            }
        };
        auto store = [&](int buf) {
#pragma unroll
            for (int i = 0; i < KLOADS; ++i) {
                const int s = tid + i * NTHR;
                const int row = s / KSEG, sg = s - (s / KSEG) * KSEG;
                if (s < 64 * KSEG) {
                    *reinterpret_cast<uint4*>(&sK[buf][row * KROW + sg * 8]) = kst[i];
                    *reinterpret_cast<uint4*>(&sV[buf][row * KROW + sg * 8]) = vst[i];
                }
            }
        };

        load(0);
        store(0);
        __syncthreads();
        for (int it = 0; it < iters; ++it) {
            const int buf = it & 1;
            if (it + 1 < iters) load(it + 1);
            const int u = it / nch, ch = it - (it / nch) * nch;
            const int ml = sList[u];
            const int m = seg0 + ml;
            const int kb = m * a.kvb - a.kv_pad + ch * 64;
            const int rem = a.kvb - ch * 64;
            uint32_t mk[TPW];
            bool anyt = false;
#pragma unroll
            for (int tt = 0; tt < TPW; ++tt) {
                mk[tt] = __builtin_amdgcn_readfirstlane(sMask[wave * TPW + tt][ml]);
                anyt |= mk[tt] != 0u;
            }
            if (anyt) {
                f32x16 s[TPW][2];
#pragma unroll
                for (int tt = 0; tt < TPW; ++tt)
#pragma unroll
                    for (int sb = 0; sb < 2; ++sb)
#pragma unroll
                        for (int i = 0; i < 16; ++i) s[tt][sb][i] = 0.f;
                const uint16_t* kbase = &sK[buf][0];
                // both 32-key halves in one loop: two independent MFMA chains
                // (keys past a short chunk are zero rows, masked below)
#pragma unroll
                for (int ks = 0; ks < KS; ++ks) {
                    const uint4 a0 = *reinterpret_cast<const uint4*>(kbase + (lane & 31) * KROW + ks * 16 + hf * 8);
                    const uint4 a1 =
                        *reinterpret_cast<const uint4*>(kbase + (32 + (lane & 31)) * KROW + ks * 16 + hf * 8);
#pragma unroll
                    for (int tt = 0; tt < TPW; ++tt)
                        if (mk[tt]) {
                            s[tt][0] = E::mma(a0, qf[tt][ks], s[tt][0]);
                            s[tt][1] = E::mma(a1, qf[tt][ks], s[tt][1]);
                        }
                }
#pragma unroll
                for (int tt = 0; tt < TPW; ++tt) {
                    if (!mk[tt]) continue;
                    const bool colok = (mk[tt] >> (lane & 31)) & 1u;
                    const int klo = colok ? max(0, -kb) : 64;
                    const int khi = colok ? min(min(rem, 64), a.N - kb) : 0;
                    const unsigned kw = (unsigned)max(khi - klo, 0);  // a chunk past N has khi < klo
                    float mx = -FTA_INF;
#pragma unroll
                    for (int sb = 0; sb < 2; ++sb)
#pragma unroll
                        for (int i = 0; i < 16; ++i) {
                            const int rel = sb * 32 + c_row(i, lane);
                            const float v = ((unsigned)(rel - klo) < kw) ? s[tt][sb][i] : -FTA_INF;
                            s[tt][sb][i] = v;
                            mx = fmaxf(mx, v);
                        }
                    mx = fmaxf(mx, fta_xor32(mx));
                    const float mn = fmaxf(m_run[tt], mx);
                    const bool grow = (mn - m_run[tt]) * a.c > 8.f;
                    if (__ballot(grow) != 0ull) {
                        const float alpha = grow ? fta_exp2((m_run[tt] - mn) * a.c) : 1.f;
#pragma unroll
                        for (int dt = 0; dt < DT32; ++dt)
#pragma unroll
                            for (int i = 0; i < 16; ++i) oacc[tt][dt][i] *= alpha;
                        l_run[tt] *= alpha;
                        if (grow) m_run[tt] = mn;
                    }
                    const float mc = (m_run[tt] == -FTA_INF) ? 0.f : m_run[tt] * a.c;
                    float ls = 0.f;
                    uint4 pf[4];
#pragma unroll
                    for (int ks = 0; ks < 4; ++ks) {
                        float pv[8];
#pragma unroll
                        for (int e = 0; e < 8; ++e) {
                            pv[e] = fta_exp2(fmaf(s[tt][ks >> 1][8 * (ks & 1) + e], a.c, -mc));
                            ls += pv[e];
                        }
                        pf[ks] = make_uint4(E::pack2(pv[0], pv[1]), E::pack2(pv[2], pv[3]), E::pack2(pv[4], pv[5]),
                                            E::pack2(pv[6], pv[7]));
                    }
                    l_run[tt] += ls;
                    const uint16_t* vbase = &sV[buf][0];
#pragma unroll
                    for (int ks = 0; ks < 4; ++ks) {
#pragma unroll
                        for (int dt = 0; dt < DT32; ++dt) {
                            const uint4 vf = fta_tr_frag(vbase, KROW, ks * 16, dt * 32, lane);
                            oacc[tt][dt] = E::mma(vf, pf[ks], oacc[tt][dt]);
                        }
                    }
                }
            }
            if (it + 1 < iters) store(buf ^ 1);
            __syncthreads();
        }
    }

    // finalize: O = O^T / L, lse = ln(sum) + max
#pragma unroll
    for (int tt = 0; tt < TPW; ++tt) {
        const float L = l_run[tt] + fta_xor32(l_run[tt]);
        const float inv = (L > 0.f) ? 1.f / L : 0.f;
        const int t = p0 + 32 * (wave * TPW + tt) + (lane & 31) - a.q_pad;
        if (t < 0 || t >= a.N) continue;
        if (lane < 32)
            a.lse[(int64_t)bh * a.N + t] =
                (L > 0.f) ? (fmaf(m_run[tt], a.c, fta_log2(L))) * 0.69314718055994531f : -FTA_INF;
        uint16_t* op = a.out0 + b * a.o0_sb + h * a.o0_sh + (int64_t)t * a.o0_sn;
#pragma unroll
        for (int dt = 0; dt < DT32; ++dt)
#pragma unroll
            for (int i = 0; i < 16; i += 4) {
                const int d = dt * 32 + c_row(i, lane);
                if (d < a.Dreal) {
                    uint2 w;
                    w.x = E::pack2(oacc[tt][dt][i] * inv, oacc[tt][dt][i + 1] * inv);
                    w.y = E::pack2(oacc[tt][dt][i + 2] * inv, oacc[tt][dt][i + 3] * inv);
                    *reinterpret_cast<uint2*>(op + d) = w;
                }
            }
    }
}

// ----------------------------------------------------------------------------
// Forward, pipelined (D = 64 and 128).  Same tiling and arithmetic as
// fta_sparse_fwd_kernel with one tile per wave, but the 64-key K and V chunks
// are gathered by LDS DMA (global_load_lds_dwordx4) into NST stage buffers in
// the swizzled row layout, NST - 1 chunks ahead of the MFMAs, so the gather
// latency is hidden behind the work of the chunks in flight and no registers
// stage the copies.
// ----------------------------------------------------------------------------
template <int D, int NW>
struct FwdPipeShape {
    static constexpr int QSEG = D / 8;
    static constexpr int SLOTS = 64 * QSEG;         // 16-byte slots per 64-row tensor chunk
    static constexpr int LQ = SLOTS / (64 * NW);    // DMA instructions per wave per tensor
    static constexpr int TEN_B = SLOTS * 16;        // bytes per tensor chunk
    static constexpr int STAGE_B = 2 * TEN_B;       // K then V
    static constexpr int NST = (3 * STAGE_B <= 96 * 1024 && D <= 64) ? 4 : 3;
    static_assert(SLOTS % (64 * NW) == 0, "whole DMA instructions per wave");
    static_assert(NST * STAGE_B + NW * kSeg * 4 + kSeg * 4 <= 150 * 1024, "LDS budget");
};

// Empty asm with every fragment as a read-write VGPR operand: all loads into
// `f` complete before it, and none can be moved below it.
typedef unsigned int fta_u32x4v __attribute__((ext_vector_type(4)));
template <int KS>
__device__ __forceinline__ void fta_pin_frags(uint4 (&f)[2][KS]) {
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int k = 0; k < KS; k += 4) {
            fta_u32x4v x0 = __builtin_bit_cast(fta_u32x4v, f[h][k]);
            fta_u32x4v x1 = __builtin_bit_cast(fta_u32x4v, f[h][(k + 1) % KS]);
            fta_u32x4v x2 = __builtin_bit_cast(fta_u32x4v, f[h][(k + 2) % KS]);
            fta_u32x4v x3 = __builtin_bit_cast(fta_u32x4v, f[h][(k + 3) % KS]);
            asm volatile("" : "+v"(x0), "+v"(x1), "+v"(x2), "+v"(x3));
            f[h][k] = __builtin_bit_cast(uint4, x0);
            if (k + 1 < KS) f[h][k + 1] = __builtin_bit_cast(uint4, x1);
            if (k + 2 < KS) f[h][k + 2] = __builtin_bit_cast(uint4, x2);
            if (k + 3 < KS) f[h][k + 3] = __builtin_bit_cast(uint4, x3);
        }
}

// SPLIT: workgroup (tiles, part sp) walks union positions [sp U / nsplit,
// (sp + 1) U / nsplit) of each mask segment and writes its unnormalised partial
// output, running max and sum instead of o and lse.
template <int DT, int D, int NW, bool SPLIT>
__global__ __launch_bounds__(NW * 64, 1) void fta_sparse_fwd_pipe_kernel(AttnArgs a) {
    using E = Elem<DT>;
    using Sh = FwdPipeShape<D, NW>;
    constexpr int QSEG = Sh::QSEG, LQ = Sh::LQ, NST = Sh::NST;
    using SW = FtaSwz<QSEG>;
    constexpr int T = NW;
    constexpr int KS = D / 16;
    constexpr int DT32 = D / 32;
    __shared__ __align__(1024) unsigned char sStage[NST][Sh::STAGE_B];
    __shared__ uint32_t sMask[T][kSeg];
    __shared__ int sList[kSeg];
    __shared__ int s_tmp[8];

    const int wgi = fta_xcd_remap(blockIdx.x, a.total);
    int hp, wq, sp = 0;  // head position, tile group, part
    if constexpr (SPLIT) {
        const int per = a.wg_per_bh * a.nsplit;
        hp = wgi / per;
        const int r = wgi - hp * per;
        wq = r / a.nsplit;
        sp = r - wq * a.nsplit;
    } else {
        hp = wgi / a.wg_per_bh;
        wq = wgi - hp * a.wg_per_bh;
    }
    const int bh = a.head_perm ? a.head_perm[hp] : hp;  // (b, h)
    const int b = bh / a.H, h = bh - (bh / a.H) * a.H;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int hf = lane >> 5;
    const int p0 = wq * 32 * T;

    const uint16_t* qp = a.q + b * a.q_sb + h * a.q_sh;
    const uint16_t* kp = a.k + b * a.k_sb + (h / a.G) * a.k_sh;
    const uint16_t* vp = a.v + b * a.v_sb + (h / a.G) * a.v_sh;

    uint4 qf[KS];
    {
        const int t = p0 + 32 * wave + (lane & 31) - a.q_pad;
        const bool ok = t >= 0 && t < a.N;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            const int d = ks * 16 + hf * 8;
            qf[ks] = (ok && d < a.Dreal) ? *reinterpret_cast<const uint4*>(qp + (int64_t)t * a.q_sn + d) : fta_zero4();
        }
    }
    // the Q loads stay in flight while the masks are built (their wait is before the
    // first DMA below: the DMAs are invisible to the compiler's wait counting)

    f32x16 oacc[DT32];
#pragma unroll
    for (int dt = 0; dt < DT32; ++dt)
#pragma unroll
        for (int i = 0; i < 16; ++i) oacc[dt][i] = 0.f;
    float m_run = -FTA_INF, l_run = 0.f;

    // Per-lane DMA sources: instruction i of this wave fills the 1 KB block
    // i * NW + wave of each tensor chunk; koff / voff = row * stride + column.
    int koff[LQ], voff[LQ];
#pragma unroll
    for (int i = 0; i < LQ; ++i) {
        const int sidx = (i * NW + wave) * 64 + lane;
        const int row = sidx / QSEG;
        int j = SW::slot(row, sidx - row * QSEG);
        if (j * 8 >= a.Dreal) j = 0;  // columns past D: zero q columns / outputs never stored
        koff[i] = row * (int)a.k_sn + j * 8;
        voff[i] = row * (int)a.v_sn + j * 8;
    }
    const uint32_t lds0 = fta_lds_addr(&sStage[0][0]);
    const int nch = (a.kvb + 63) >> 6;

    for (int seg0 = 0; seg0 < a.Mkv; seg0 += kSeg) {
        const int segn = min(kSeg, a.Mkv - seg0);
        const int U = fta_build_q_masks<T>(a, bh, p0, seg0, segn, sMask, sList, s_tmp);
        int u_lo = 0, u_n = U;  // this part's union positions (workgroup-uniform)
        if constexpr (SPLIT) {
            u_lo = (U * sp) / a.nsplit;
            u_n = (U * (sp + 1)) / a.nsplit - u_lo;
        }
        // no wave reads sMask / sList below when the part is empty
        if (u_n == 0) continue;
        const int iters = u_n * nch;

        // gather chunk `it` (64 keys of union block it / nch) into stage buffer st
        auto issue = [&](int st, int it) {
            const uint32_t sb = lds0 + st * Sh::STAGE_B;
            const int u = u_lo + it / nch, ch = it - (it / nch) * nch;
            const int m = __builtin_amdgcn_readfirstlane(seg0 + sList[u]);
            const int kb = m * a.kvb - a.kv_pad + ch * 64;
            const int rem = a.kvb - ch * 64;
            if (kb >= 0 && kb + 64 <= a.N && rem >= 64) {
                const uint16_t* kbp = kp + (int64_t)kb * a.k_sn;
                const uint16_t* vbp = vp + (int64_t)kb * a.v_sn;
#pragma unroll
                for (int i = 0; i < LQ; ++i) fta_dma16_at(kbp + koff[i], sb + (i * NW + wave) * 1024);
#pragma unroll
                for (int i = 0; i < LQ; ++i) fta_dma16_at(vbp + voff[i], sb + Sh::TEN_B + (i * NW + wave) * 1024);
            } else {  // chunk at a sequence / block edge: clamp rows into [0, N) (masked below)
#pragma unroll
                for (int i = 0; i < LQ; ++i) {
                    const int sidx = (i * NW + wave) * 64 + lane;
                    const int row = sidx / QSEG;
                    int j = SW::slot(row, sidx - row * QSEG);
                    if (j * 8 >= a.Dreal) j = 0;
                    const int t = min(max(kb + row, 0), a.N - 1);
                    fta_dma16_at(kp + (int64_t)t * a.k_sn + j * 8, sb + (i * NW + wave) * 1024);
                    fta_dma16_at(vp + (int64_t)t * a.v_sn + j * 8, sb + Sh::TEN_B + (i * NW + wave) * 1024);
                }
            }
        };

        fta_wait_vmcnt<0>();  // register loads complete before the DMA stream
#pragma unroll
        for (int k = 0; k < NST - 1; ++k)
            if (k < iters) issue(k, k);
        int cur = 0;
        for (int it = 0; it < iters; ++it) {
            // chunk it resident: chunks issued so far = min(iters, it + NST - 1)
            if (it + NST - 2 < iters)
                fta_wait_vmcnt<2 * LQ * (NST - 2)>();
            else
                fta_wait_vmcnt<0>();
            __syncthreads();  // chunk it visible; every wave is past chunk it - 1
            if (it + NST - 1 < iters) issue(cur == 0 ? NST - 1 : cur - 1, it + NST - 1);

            const int u = u_lo + it / nch, ch = it - (it / nch) * nch;
            const int ml = sList[u];
            const int m = seg0 + ml;
            const int kb = m * a.kvb - a.kv_pad + ch * 64;
            const int rem = a.kvb - ch * 64;
            const uint32_t mk = __builtin_amdgcn_readfirstlane(sMask[wave][ml]);
            if (mk) {
                const uint16_t* kbase = reinterpret_cast<const uint16_t*>(&sStage[cur][0]);
                const uint16_t* vbase = kbase + Sh::TEN_B / 2;
                f32x16 s[2];
#pragma unroll
                for (int sb = 0; sb < 2; ++sb)
#pragma unroll
                    for (int i = 0; i < 16; ++i) s[sb][i] = 0.f;
                // all K fragments of the chunk first, then the MFMAs: one LDS
                // latency per chunk instead of one per MFMA
                uint4 ka[2][KS];
#pragma unroll
                for (int ks = 0; ks < KS; ++ks) {
                    ka[0][ks] = *reinterpret_cast<const uint4*>(kbase + SW::off(lane & 31, 2 * ks + hf));
                    ka[1][ks] = *reinterpret_cast<const uint4*>(kbase + SW::off(32 + (lane & 31), 2 * ks + hf));
                }
                // the empty asm takes every fragment as an operand, so the loads
                // cannot sink to their MFMAs (which exposes one LDS latency per MFMA)
                fta_pin_frags<KS>(ka);
#pragma unroll
                for (int ks = 0; ks < KS; ++ks) {
                    s[0] = E::mma(ka[0][ks], qf[ks], s[0]);
                    s[1] = E::mma(ka[1][ks], qf[ks], s[1]);
                }
                // valid keys of the chunk: [klo, khi) relative to kb (wave-uniform).
                // Keys outside it get -inf scores in place (chunks at a sequence end
                // or past a short block only).  A lane whose query column is not
                // selected keeps its scores but takes no part: its chunk maximum is
                // -inf and its exps use an infinite offset (exactly 0).
                const int klo = max(0, -kb), khi = min(min(rem, 64), a.N - kb);
                if (klo > 0 || khi < 64) {
                    const unsigned kw = (unsigned)max(khi - klo, 0);  // a chunk past N has khi < klo
#pragma unroll
                    for (int sb = 0; sb < 2; ++sb)
#pragma unroll
                        for (int i = 0; i < 16; ++i) {
                            const int rel = sb * 32 + c_row(i, lane);
                            s[sb][i] = ((unsigned)(rel - klo) < kw) ? s[sb][i] : -FTA_INF;
                        }
                }
                const bool colok = (mk >> (lane & 31)) & 1u;
                float mx = s[0][0];
#pragma unroll
                for (int sb = 0; sb < 2; ++sb)
#pragma unroll
                    for (int i = (sb == 0); i < 16; ++i) mx = fmaxf(mx, s[sb][i]);
                mx = colok ? mx : -FTA_INF;
                mx = fmaxf(mx, fta_xor32(mx));
                const float mn = fmaxf(m_run, mx);
                const bool grow = (mn - m_run) * a.c > 8.f;
                if (__ballot(grow) != 0ull) {
                    const float alpha = grow ? fta_exp2((m_run - mn) * a.c) : 1.f;
#pragma unroll
                    for (int dt = 0; dt < DT32; ++dt)
#pragma unroll
                        for (int i = 0; i < 16; ++i) oacc[dt][i] *= alpha;
                    l_run *= alpha;
                    if (grow) m_run = mn;
                }
                const float mc = !colok ? FTA_INF : (m_run == -FTA_INF) ? 0.f : m_run * a.c;
                float ls = 0.f;
                uint4 pf[4];
#pragma unroll
                for (int ks = 0; ks < 4; ++ks) {
                    float pv[8];
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        pv[e] = fta_exp2(fmaf(s[ks >> 1][8 * (ks & 1) + e], a.c, -mc));
                        ls += pv[e];
                    }
                    pf[ks] = make_uint4(E::pack2(pv[0], pv[1]), E::pack2(pv[2], pv[3]), E::pack2(pv[4], pv[5]),
                                        E::pack2(pv[6], pv[7]));
                }
                l_run += ls;
#pragma unroll
                for (int ks = 0; ks < 4; ++ks) {
#pragma unroll
                    for (int dt = 0; dt < DT32; ++dt) {
                        const uint4 vf = fta_tr_frag_sw<QSEG>(vbase, ks * 16, dt * 32, lane);
                        oacc[dt] = E::mma(vf, pf[ks], oacc[dt]);
                    }
                }
            }
            cur = (cur == NST - 1) ? 0 : cur + 1;
        }
        __syncthreads();  // every wave is done with sMask / sList before the next segment rebuilds them
    }

    // finalize: O = O^T / L, lse = ln(sum) + max
    const float L = l_run + fta_xor32(l_run);
    if constexpr (SPLIT) {
        // the part's unnormalised O, its running max and sum, by padded position
        const int p = p0 + 32 * wave + (lane & 31);
        if (p >= a.npq) return;
        const int64_t row = ((int64_t)sp * a.nbh + bh) * a.npq + p;
        if (lane < 32) a.part_ml[row] = make_float2(m_run, L);
        float* po = a.part_o + row * D;
#pragma unroll
        for (int dt = 0; dt < DT32; ++dt)
#pragma unroll
            for (int i = 0; i < 16; i += 4)
                *reinterpret_cast<float4*>(po + dt * 32 + c_row(i, lane)) =
                    make_float4(oacc[dt][i], oacc[dt][i + 1], oacc[dt][i + 2], oacc[dt][i + 3]);
        return;
    }
    const float inv = (L > 0.f) ? 1.f / L : 0.f;
    const int t = p0 + 32 * wave + (lane & 31) - a.q_pad;
    if (t < 0 || t >= a.N) return;
    if (lane < 32)
        a.lse[(int64_t)bh * a.N + t] = (L > 0.f) ? (fmaf(m_run, a.c, fta_log2(L))) * 0.69314718055994531f : -FTA_INF;
    uint16_t* op = a.out0 + b * a.o0_sb + h * a.o0_sh + (int64_t)t * a.o0_sn;
#pragma unroll
    for (int dt = 0; dt < DT32; ++dt)
#pragma unroll
        for (int i = 0; i < 16; i += 4) {
            const int d = dt * 32 + c_row(i, lane);
            if (d < a.Dreal) {
                uint2 w;
                w.x = E::pack2(oacc[dt][i] * inv, oacc[dt][i + 1] * inv);
                w.y = E::pack2(oacc[dt][i + 2] * inv, oacc[dt][i + 3] * inv);
                *reinterpret_cast<uint2*>(op + d) = w;
            }
        }
}

// Merge of the forward's split parts: one thread per (b·h, query, 8 columns).
// m = max over the parts with a positive sum; O = sum_p O_p 2^{c (m_p - m)} / L,
// L = sum_p L_p 2^{c (m_p - m)}, lse = (c m + log2 L) ln 2 (-inf, O = 0 for a
// query with no selected key, as in the unsplit kernel).
template <int DT, int D>
__global__ __launch_bounds__(256) void fta_fwd_combine_kernel(AttnArgs a) {
    using E = Elem<DT>;
    constexpr int DC = D / 8;
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (int64_t)a.nbh * a.N * DC) return;
    const int dc = (int)(idx % DC);
    const int64_t rest = idx / DC;
    const int t = (int)(rest % a.N), bh = (int)(rest / a.N);
    const int d0 = dc * 8;
    if (d0 >= a.Dreal && dc != 0) return;
    const int p = t + a.q_pad;
    float m = -FTA_INF;
    for (int sp = 0; sp < a.nsplit; ++sp) {
        const float2 ml = a.part_ml[((int64_t)sp * a.nbh + bh) * a.npq + p];
        if (ml.y > 0.f) m = fmaxf(m, ml.x);
    }
    float L = 0.f, o[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int sp = 0; sp < a.nsplit; ++sp) {
        const int64_t row = ((int64_t)sp * a.nbh + bh) * a.npq + p;
        const float2 ml = a.part_ml[row];
        if (!(ml.y > 0.f)) continue;
        const float w = fta_exp2((ml.x - m) * a.c);
        L = fmaf(ml.y, w, L);
        const float4 x0 = *reinterpret_cast<const float4*>(a.part_o + row * D + d0);
        const float4 x1 = *reinterpret_cast<const float4*>(a.part_o + row * D + d0 + 4);
        o[0] = fmaf(x0.x, w, o[0]);
        o[1] = fmaf(x0.y, w, o[1]);
        o[2] = fmaf(x0.z, w, o[2]);
        o[3] = fmaf(x0.w, w, o[3]);
        o[4] = fmaf(x1.x, w, o[4]);
        o[5] = fmaf(x1.y, w, o[5]);
        o[6] = fmaf(x1.z, w, o[6]);
        o[7] = fmaf(x1.w, w, o[7]);
    }
    const int b = bh / a.H, h = bh - (bh / a.H) * a.H;
    if (dc == 0)
        a.lse[(int64_t)bh * a.N + t] = (L > 0.f) ? fmaf(m, a.c, fta_log2(L)) * 0.69314718055994531f : -FTA_INF;
    if (d0 >= a.Dreal) return;
    const float inv = (L > 0.f) ? 1.f / L : 0.f;
    uint16_t* op = a.out0 + b * a.o0_sb + h * a.o0_sh + (int64_t)t * a.o0_sn + d0;
    *reinterpret_cast<uint2*>(op) = make_uint2(E::pack2(o[0] * inv, o[1] * inv), E::pack2(o[2] * inv, o[3] * inv));
    *reinterpret_cast<uint2*>(op + 4) = make_uint2(E::pack2(o[4] * inv, o[5] * inv), E::pack2(o[6] * inv, o[7] * inv));
}

// ----------------------------------------------------------------------------
// dQ.  Same tiling as the forward (one tile per wave).  Per union KV chunk:
//   S^T = K Q^T, P^T = 2^{c S^T - lse2}, dP^T = V dO^T, dS^T = P^T (dP^T - delta),
//   dQ^T += K^T dS^T  (K^T from the T layout).
// ----------------------------------------------------------------------------
template <int DT, int D, int NW, bool SPLIT>
__global__ __launch_bounds__(NW * 64, 1) void fta_sparse_dq_kernel(AttnArgs a) {
    using E = Elem<DT>;
    constexpr int NB = (D <= 160) ? 2 : 1;  // LDS buffers (D = 256 single-buffers to fit 160 KB)
    constexpr int NTHR = NW * 64;
    constexpr int T = NW;
    constexpr int KS = D / 16;
    constexpr int DT32 = D / 32;
    constexpr int KROW = D + 8;
    constexpr int KSEG = D / 8;
    constexpr int KLOADS = (64 * KSEG + NTHR - 1) / NTHR;
    __shared__ __align__(16) uint16_t sK[NB][64 * KROW];
    __shared__ __align__(16) uint16_t sV[NB][64 * KROW];
    __shared__ uint32_t sMask[T][kSeg];
    __shared__ int sList[kSeg];
    __shared__ int s_tmp[8];

    const int wgi = fta_xcd_remap(blockIdx.x, a.total);
    int bh, wq, sp = 0;  // (b, h), tile group, part (as in fta_sparse_dq_pipe_kernel)
    if constexpr (SPLIT) {
        const int per = a.wg_per_bh * a.nsplit;
        bh = wgi / per;
        const int r = wgi - bh * per;
        wq = r / a.nsplit;
        sp = r - wq * a.nsplit;
    } else {
        bh = wgi / a.wg_per_bh;
        wq = wgi - bh * a.wg_per_bh;
    }
    const int b = bh / a.H, h = bh - (bh / a.H) * a.H;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int hf = lane >> 5;
    const int p0 = wq * 32 * T;

    const uint16_t* qp = a.q + b * a.q_sb + h * a.q_sh;
    const uint16_t* kp = a.k + b * a.k_sb + (h / a.G) * a.k_sh;
    const uint16_t* vp = a.v + b * a.v_sb + (h / a.G) * a.v_sh;
    const uint16_t* dp = a.dout + b * a.d_sb + h * a.d_sh;

    const int tq = p0 + 32 * wave + (lane & 31) - a.q_pad;
    const bool qok = tq >= 0 && tq < a.N;
    uint4 qf[KS], df[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
        const int d = ks * 16 + hf * 8;
        const bool ok = qok && d < a.Dreal;
        qf[ks] = ok ? *reinterpret_cast<const uint4*>(qp + (int64_t)tq * a.q_sn + d) : fta_zero4();
        df[ks] = ok ? *reinterpret_cast<const uint4*>(dp + (int64_t)tq * a.d_sn + d) : fta_zero4();
    }
    float lse2 = -FTA_INF, dl = 0.f;
    if (qok) {
        lse2 = a.lse_in[(int64_t)bh * a.N + tq] * 1.4426950408889634f;
        dl = a.delta_in[(int64_t)bh * a.N + tq];
    }
    const bool rowlive = lse2 != -FTA_INF;

    f32x16 acc[DT32];
#pragma unroll
    for (int dt = 0; dt < DT32; ++dt)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[dt][i] = 0.f;

    const int nch = (a.kvb + 63) >> 6;
    uint4 kst[KLOADS], vst[KLOADS];

    for (int seg0 = 0; seg0 < a.Mkv; seg0 += kSeg) {
        const int segn = min(kSeg, a.Mkv - seg0);
        const int U = fta_build_q_masks<T>(a, bh, p0, seg0, segn, sMask, sList, s_tmp);
        int u_lo = 0, u_n = U;  // this part's union positions (workgroup-uniform)
        if constexpr (SPLIT) {
            u_lo = (U * sp) / a.nsplit;
            u_n = (U * (sp + 1)) / a.nsplit - u_lo;
        }
        if (u_n == 0) continue;
        const int iters = u_n * nch;
        auto load = [&](int it) {
            const int u = u_lo + it / nch, ch = it - (it / nch) * nch;
            const int m = seg0 + sList[u];
            const int kb = m * a.kvb - a.kv_pad + ch * 64;
            const int rem = a.kvb - ch * 64;
#pragma unroll
            for (int i = 0; i < KLOADS; ++i) {
                const int s = tid + i * NTHR;
                const int row = s / KSEG, sg = s - (s / KSEG) * KSEG;
                const int t = kb + row;
                const bool ok = s < 64 * KSEG && row < rem && t >= 0 && t < a.N && sg * 8 < a.Dreal;
                kst[i] = ok ? *reinterpret_cast<const uint4*>(kp + (int64_t)t * a.k_sn + sg * 8) : fta_zero4();
                vst[i] = ok ? *reinterpret_cast<const uint4*>(vp + (int64_t)t * a.v_sn + sg * 8) : fta_zero4();
            }
        };
        auto store = [&](int buf) {
#pragma unroll
            for (int i = 0; i < KLOADS; ++i) {
                const int s = tid + i * NTHR;
                const int row = s / KSEG, sg = s - (s / KSEG) * KSEG;
                if (s < 64 * KSEG) {
                    *reinterpret_cast<uint4*>(&sK[buf][row * KROW + sg * 8]) = kst[i];
                    *reinterpret_cast<uint4*>(&sV[buf][row * KROW + sg * 8]) = vst[i];
                }
            }
        };

        load(0);
        store(0);
        __syncthreads();
        for (int it = 0; it < iters; ++it) {
            const int buf = (NB == 2) ? (it & 1) : 0;
            if (it + 1 < iters) load(it + 1);
            const int u = u_lo + it / nch, ch = it - (it / nch) * nch;
            const int ml = sList[u];
            const int m = seg0 + ml;
            const int kb = m * a.kvb - a.kv_pad + ch * 64;
            const int rem = a.kvb - ch * 64;
            const bool two = rem > 32;
            const uint32_t mk = __builtin_amdgcn_readfirstlane(sMask[wave][ml]);
            if (mk) {
                f32x16 s[2], dpv[2];
#pragma unroll
                for (int sb = 0; sb < 2; ++sb)
#pragma unroll
                    for (int i = 0; i < 16; ++i) {
                        s[sb][i] = 0.f;
                        dpv[sb][i] = 0.f;
                    }
                const uint16_t* kbase = &sK[buf][0];
                const uint16_t* vbase = &sV[buf][0];
                const int nsb = two ? 2 : 1;
#pragma unroll
                for (int sb = 0; sb < 2; ++sb) {
                    if (sb >= nsb) break;
#pragma unroll
                    for (int ks = 0; ks < KS; ++ks) {
                        const int off = (sb * 32 + (lane & 31)) * KROW + ks * 16 + hf * 8;
                        s[sb] = E::mma(*reinterpret_cast<const uint4*>(kbase + off), qf[ks], s[sb]);
                        dpv[sb] = E::mma(*reinterpret_cast<const uint4*>(vbase + off), df[ks], dpv[sb]);
                    }
                }
                // valid keys [klo, khi) relative to kb; a lane whose query column
                // is not selected gets the empty range (branch-free masking)
                const bool colok = rowlive && ((mk >> (lane & 31)) & 1u);
                const int klo = colok ? max(0, -kb) : 64;
                const int khi = colok ? min(min(rem, 64), a.N - kb) : 0;
                const unsigned kw = (unsigned)max(khi - klo, 0);  // a chunk past N has khi < klo
                uint4 dsf[4];
#pragma unroll
                for (int ks = 0; ks < 4; ++ks) {
                    float dsv[8];
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        const int sb = ks >> 1, i = 8 * (ks & 1) + e;
                        const int rel = sb * 32 + c_row(i, lane);
                        const bool ok = (unsigned)(rel - klo) < kw;
                        const float ex = fta_exp2(fmaf(s[sb][i], a.c, -lse2));
                        const float p = ok ? ex : 0.f;
                        dsv[e] = p * (dpv[sb][i] - dl);
                    }
                    dsf[ks] = make_uint4(E::pack2(dsv[0], dsv[1]), E::pack2(dsv[2], dsv[3]),
                                         E::pack2(dsv[4], dsv[5]), E::pack2(dsv[6], dsv[7]));
                }
                const uint16_t* tbase = &sK[buf][0];
                const int nks = two ? 4 : 2;
#pragma unroll
                for (int ks = 0; ks < 4; ++ks) {
                    if (ks >= nks) break;
#pragma unroll
                    for (int dt = 0; dt < DT32; ++dt) {
                        acc[dt] = E::mma(fta_tr_frag(tbase, KROW, ks * 16, dt * 32, lane), dsf[ks], acc[dt]);
                    }
                }
            }
            if (NB == 1) __syncthreads();
            if (it + 1 < iters) store((NB == 2) ? (buf ^ 1) : 0);
            __syncthreads();
        }
    }

    if constexpr (SPLIT) {
        // the part's unscaled dQ, by padded position (rows outside [0, N) hold zeros)
        const int p = p0 + 32 * wave + (lane & 31);
        if (p >= a.npq) return;
        float* po = a.part_o + (((int64_t)sp * a.nbh + bh) * a.npq + p) * D;
#pragma unroll
        for (int dt = 0; dt < DT32; ++dt)
#pragma unroll
            for (int i = 0; i < 16; i += 4)
                *reinterpret_cast<float4*>(po + dt * 32 + c_row(i, lane)) =
                    make_float4(acc[dt][i], acc[dt][i + 1], acc[dt][i + 2], acc[dt][i + 3]);
        return;
    }
    if (!qok) return;
    uint16_t* op = a.out0 + b * a.o0_sb + h * a.o0_sh + (int64_t)tq * a.o0_sn;
#pragma unroll
    for (int dt = 0; dt < DT32; ++dt)
#pragma unroll
        for (int i = 0; i < 16; i += 4) {
            const int d = dt * 32 + c_row(i, lane);
            if (d < a.Dreal) {
                uint2 w;
                w.x = E::pack2(acc[dt][i] * a.scale, acc[dt][i + 1] * a.scale);
                w.y = E::pack2(acc[dt][i + 2] * a.scale, acc[dt][i + 3] * a.scale);
                *reinterpret_cast<uint2*>(op + d) = w;
            }
        }
}

// ----------------------------------------------------------------------------
// dQ, pipelined (D = 64 and 128).  The arithmetic of fta_sparse_dq_kernel; the
// 64-key K and V chunks are gathered by LDS DMA into NST swizzled stage buffers
// (as in fta_sparse_fwd_pipe_kernel), NST - 1 chunks ahead, so the gather
// latency is hidden and the operand reads (K and V rows, K^T transposed) are
// free of LDS bank conflicts.
// SPLIT: workgroup (tiles, part sp) walks union positions [sp U / nsplit,
// (sp + 1) U / nsplit) of each mask segment and writes its unscaled fp32 dQ
// partial; fta_dq_combine_kernel adds the parts (dQ is linear in them).
// ----------------------------------------------------------------------------
template <int DT, int D, bool SPLIT>
__global__ __launch_bounds__(512, 1) void fta_sparse_dq_pipe_kernel(AttnArgs a) {
    using E = Elem<DT>;
    constexpr int NW = 8, T = 8;
    using Sh = FwdPipeShape<D, NW>;
    constexpr int QSEG = Sh::QSEG, LQ = Sh::LQ, NST = Sh::NST;
    using SW = FtaSwz<QSEG>;
    constexpr int KS = D / 16;
    constexpr int DT32 = D / 32;
    __shared__ __align__(1024) unsigned char sStage[NST][Sh::STAGE_B];
    __shared__ uint32_t sMask[T][kSeg];
    __shared__ int sList[kSeg];
    __shared__ int s_tmp[8];

    const int wgi = fta_xcd_remap(blockIdx.x, a.total);
    int hp, wq, sp = 0;  // head position, tile group, part
    if constexpr (SPLIT) {
        const int per = a.wg_per_bh * a.nsplit;
        hp = wgi / per;
        const int r = wgi - hp * per;
        wq = r / a.nsplit;
        sp = r - wq * a.nsplit;
    } else {
        hp = wgi / a.wg_per_bh;
        wq = wgi - hp * a.wg_per_bh;
    }
    const int bh = a.head_perm ? a.head_perm[hp] : hp;  // (b, h)
    const int b = bh / a.H, h = bh - (bh / a.H) * a.H;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int hf = lane >> 5;
    const int p0 = wq * 32 * T;

    const uint16_t* qp = a.q + b * a.q_sb + h * a.q_sh;
    const uint16_t* kp = a.k + b * a.k_sb + (h / a.G) * a.k_sh;
    const uint16_t* vp = a.v + b * a.v_sb + (h / a.G) * a.v_sh;
    const uint16_t* dp = a.dout + b * a.d_sb + h * a.d_sh;

    const int tq = p0 + 32 * wave + (lane & 31) - a.q_pad;
    const bool qok = tq >= 0 && tq < a.N;
    uint4 qf[KS], df[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
        const int d = ks * 16 + hf * 8;
        const bool ok = qok && d < a.Dreal;
        qf[ks] = ok ? *reinterpret_cast<const uint4*>(qp + (int64_t)tq * a.q_sn + d) : fta_zero4();
        df[ks] = ok ? *reinterpret_cast<const uint4*>(dp + (int64_t)tq * a.d_sn + d) : fta_zero4();
    }
    float lse2 = -FTA_INF, dl = 0.f;
    if (qok) {
        lse2 = a.lse_in[(int64_t)bh * a.N + tq] * 1.4426950408889634f;
        dl = a.delta_in[(int64_t)bh * a.N + tq];
    }
    const bool rowlive = lse2 != -FTA_INF;
    // the Q / dO loads stay in flight while the masks are built (their wait is before
    // the first DMA below: the DMAs are invisible to the compiler's wait counting)

    f32x16 acc[DT32];
#pragma unroll
    for (int dt = 0; dt < DT32; ++dt)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[dt][i] = 0.f;

    // Per-lane DMA sources: instruction i of this wave fills the 1 KB block
    // i * NW + wave of each tensor chunk; koff / voff = row * stride + column.
    int koff[LQ], voff[LQ];
#pragma unroll
    for (int i = 0; i < LQ; ++i) {
        const int sidx = (i * NW + wave) * 64 + lane;
        const int row = sidx / QSEG;
        int j = SW::slot(row, sidx - row * QSEG);
        if (j * 8 >= a.Dreal) j = 0;  // columns past D: zero q / dO columns, outputs never stored
        koff[i] = row * (int)a.k_sn + j * 8;
        voff[i] = row * (int)a.v_sn + j * 8;
    }
    const uint32_t lds0 = fta_lds_addr(&sStage[0][0]);
    const int nch = (a.kvb + 63) >> 6;

    for (int seg0 = 0; seg0 < a.Mkv; seg0 += kSeg) {
        const int segn = min(kSeg, a.Mkv - seg0);
        const int U = fta_build_q_masks<T>(a, bh, p0, seg0, segn, sMask, sList, s_tmp);
        int u_lo = 0, u_n = U;  // this part's union positions (workgroup-uniform)
        if constexpr (SPLIT) {
            u_lo = (U * sp) / a.nsplit;
            u_n = (U * (sp + 1)) / a.nsplit - u_lo;
        }
        // no wave reads sMask / sList below when the part is empty
        if (u_n == 0) continue;
        const int iters = u_n * nch;

        auto issue = [&](int st, int it) {
            const uint32_t sb = lds0 + st * Sh::STAGE_B;
            const int u = u_lo + it / nch, ch = it - (it / nch) * nch;
            const int m = __builtin_amdgcn_readfirstlane(seg0 + sList[u]);
            const int kb = m * a.kvb - a.kv_pad + ch * 64;
            const int rem = a.kvb - ch * 64;
            if (kb >= 0 && kb + 64 <= a.N && rem >= 64) {
                const uint16_t* kbp = kp + (int64_t)kb * a.k_sn;
                const uint16_t* vbp = vp + (int64_t)kb * a.v_sn;
#pragma unroll
                for (int i = 0; i < LQ; ++i) fta_dma16_at(kbp + koff[i], sb + (i * NW + wave) * 1024);
#pragma unroll
                for (int i = 0; i < LQ; ++i) fta_dma16_at(vbp + voff[i], sb + Sh::TEN_B + (i * NW + wave) * 1024);
            } else {  // chunk at a sequence / block edge: clamp rows into [0, N) (masked below)
#pragma unroll
                for (int i = 0; i < LQ; ++i) {
                    const int sidx = (i * NW + wave) * 64 + lane;
                    const int row = sidx / QSEG;
                    int j = SW::slot(row, sidx - row * QSEG);
                    if (j * 8 >= a.Dreal) j = 0;
                    const int t = min(max(kb + row, 0), a.N - 1);
                    fta_dma16_at(kp + (int64_t)t * a.k_sn + j * 8, sb + (i * NW + wave) * 1024);
                    fta_dma16_at(vp + (int64_t)t * a.v_sn + j * 8, sb + Sh::TEN_B + (i * NW + wave) * 1024);
                }
            }
        };

        fta_wait_vmcnt<0>();  // register loads complete before the DMA stream
#pragma unroll
        for (int k = 0; k < NST - 1; ++k)
            if (k < iters) issue(k, k);
        int cur = 0;
        for (int it = 0; it < iters; ++it) {
            if (it + NST - 2 < iters)
                fta_wait_vmcnt<2 * LQ * (NST - 2)>();
            else
                fta_wait_vmcnt<0>();
            __syncthreads();  // chunk it visible; every wave is past chunk it - 1
            if (it + NST - 1 < iters) issue(cur == 0 ? NST - 1 : cur - 1, it + NST - 1);

            const int u = u_lo + it / nch, ch = it - (it / nch) * nch;
            const int ml = sList[u];
            const int m = seg0 + ml;
            const int kb = m * a.kvb - a.kv_pad + ch * 64;
            const int rem = a.kvb - ch * 64;
            const bool two = rem > 32;
            const uint32_t mk = __builtin_amdgcn_readfirstlane(sMask[wave][ml]);
            if (mk) {
                const uint16_t* kbase = reinterpret_cast<const uint16_t*>(&sStage[cur][0]);
                const uint16_t* vbase = kbase + Sh::TEN_B / 2;
                // A lane whose query column is not selected uses an infinite lse:
                // all its exps are exactly 0.  Keys outside [klo, khi) (chunks at
                // a sequence end, or past a short block) get -inf scores in place
                // under a wave-uniform branch; every other chunk is unmasked.
                const bool colok = rowlive && ((mk >> (lane & 31)) & 1u);
                const float lse_c = colok ? lse2 : FTA_INF;
                const int klo = max(0, -kb), khi = min(min(rem, 64), a.N - kb);
                const int nsb = two ? 2 : 1;
                uint4 dsf[4];
                // one 32-key half at a time (S and dP of one half live), the K / V
                // fragments loaded one MFMA pair ahead
#pragma unroll
                for (int sb = 0; sb < 2; ++sb) {
                    if (sb >= nsb) break;
                    f32x16 s, dpv;
#pragma unroll
                    for (int i = 0; i < 16; ++i) {
                        s[i] = 0.f;
                        dpv[i] = 0.f;
                    }
                    // rows 32 sb + r share row r's swizzle: one offset per k slot
                    const uint16_t* kh = kbase + sb * 32 * QSEG * 8;
                    const uint16_t* vh = vbase + sb * 32 * QSEG * 8;
                    uint4 kf[2], vf[2];
                    kf[0] = *reinterpret_cast<const uint4*>(kh + SW::off(lane & 31, hf));
                    vf[0] = *reinterpret_cast<const uint4*>(vh + SW::off(lane & 31, hf));
#pragma unroll
                    for (int ks = 0; ks < KS; ++ks) {
                        if (ks + 1 < KS) {
                            const int off = SW::off(lane & 31, 2 * (ks + 1) + hf);
                            kf[(ks + 1) & 1] = *reinterpret_cast<const uint4*>(kh + off);
                            vf[(ks + 1) & 1] = *reinterpret_cast<const uint4*>(vh + off);
                        }
                        s = E::mma(kf[ks & 1], qf[ks], s);
                        dpv = E::mma(vf[ks & 1], df[ks], dpv);
                    }
                    if (klo > 0 || khi < 64) {
                        const unsigned kw = (unsigned)max(khi - klo, 0);  // a chunk past N has khi < klo
#pragma unroll
                        for (int i = 0; i < 16; ++i) {
                            const int rel = sb * 32 + c_row(i, lane);
                            s[i] = ((unsigned)(rel - klo) < kw) ? s[i] : -FTA_INF;
                        }
                    }
#pragma unroll
                    for (int k2 = 0; k2 < 2; ++k2) {
                        float dsv[8];
#pragma unroll
                        for (int e = 0; e < 8; ++e) {
                            const int i = 8 * k2 + e;
                            const float p = fta_exp2(fmaf(s[i], a.c, -lse_c));
                            dsv[e] = p * (dpv[i] - dl);
                        }
                        dsf[2 * sb + k2] = make_uint4(E::pack2(dsv[0], dsv[1]), E::pack2(dsv[2], dsv[3]),
                                                      E::pack2(dsv[4], dsv[5]), E::pack2(dsv[6], dsv[7]));
                    }
                }
                const int nks = two ? 4 : 2;
#pragma unroll
                for (int ks = 0; ks < 4; ++ks) {
                    if (ks >= nks) break;
#pragma unroll
                    for (int dt = 0; dt < DT32; ++dt)
                        acc[dt] = E::mma(fta_tr_frag_sw<QSEG>(kbase, ks * 16, dt * 32, lane), dsf[ks], acc[dt]);
                }
            }
            cur = (cur == NST - 1) ? 0 : cur + 1;
        }
        __syncthreads();  // every wave is done with sMask / sList before the next segment rebuilds them
    }

    if constexpr (SPLIT) {
        // the part's unscaled dQ, by padded position (rows outside [0, N) hold zeros)
        const int p = p0 + 32 * wave + (lane & 31);
        if (p >= a.npq) return;
        float* po = a.part_o + (((int64_t)sp * a.nbh + bh) * a.npq + p) * D;
#pragma unroll
        for (int dt = 0; dt < DT32; ++dt)
#pragma unroll
            for (int i = 0; i < 16; i += 4)
                *reinterpret_cast<float4*>(po + dt * 32 + c_row(i, lane)) =
                    make_float4(acc[dt][i], acc[dt][i + 1], acc[dt][i + 2], acc[dt][i + 3]);
        return;
    }
    if (!qok) return;
    uint16_t* op = a.out0 + b * a.o0_sb + h * a.o0_sh + (int64_t)tq * a.o0_sn;
#pragma unroll
    for (int dt = 0; dt < DT32; ++dt)
#pragma unroll
        for (int i = 0; i < 16; i += 4) {
            const int d = dt * 32 + c_row(i, lane);
            if (d < a.Dreal) {
                uint2 w;
                w.x = E::pack2(acc[dt][i] * a.scale, acc[dt][i + 1] * a.scale);
                w.y = E::pack2(acc[dt][i + 2] * a.scale, acc[dt][i + 3] * a.scale);
                *reinterpret_cast<uint2*>(op + d) = w;
            }
        }
}

// Sum of the dQ kernel's split parts: one thread per (b·h, query, 8 columns);
// dQ = scale · sum_p dQ_p, parts added in order.
template <int DT, int D>
__global__ __launch_bounds__(256) void fta_dq_combine_kernel(AttnArgs a) {
    using E = Elem<DT>;
    constexpr int DC = D / 8;
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (int64_t)a.nbh * a.N * DC) return;
    const int dc = (int)(idx % DC);
    const int64_t rest = idx / DC;
    const int t = (int)(rest % a.N), bh = (int)(rest / a.N);
    const int d0 = dc * 8;
    if (d0 >= a.Dreal) return;
    const int p = t + a.q_pad;
    float o[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int sp = 0; sp < a.nsplit; ++sp) {
        const float* src = a.part_o + (((int64_t)sp * a.nbh + bh) * a.npq + p) * D + d0;
        const float4 x0 = *reinterpret_cast<const float4*>(src);
        const float4 x1 = *reinterpret_cast<const float4*>(src + 4);
        o[0] += x0.x;
        o[1] += x0.y;
        o[2] += x0.z;
        o[3] += x0.w;
        o[4] += x1.x;
        o[5] += x1.y;
        o[6] += x1.z;
        o[7] += x1.w;
    }
    const int b = bh / a.H, h = bh - (bh / a.H) * a.H;
    uint16_t* op = a.out0 + b * a.o0_sb + h * a.o0_sh + (int64_t)t * a.o0_sn + d0;
    *reinterpret_cast<uint2*>(op) =
        make_uint2(E::pack2(o[0] * a.scale, o[1] * a.scale), E::pack2(o[2] * a.scale, o[3] * a.scale));
    *reinterpret_cast<uint2*>(op + 4) =
        make_uint2(E::pack2(o[4] * a.scale, o[5] * a.scale), E::pack2(o[6] * a.scale, o[7] * a.scale));
}

// ----------------------------------------------------------------------------
// dK / dV.  WG = TT x CS waves.  The WG owns TT 32-key tiles (consecutive
// (KV block, 32-key sub-tile) pairs); wave w works on tile w % TT and chunk
// slot w / TT.  Column masks over 32-query chunks come from the membership
// bitmap; the union of the tiles' chunks is walked CS chunks per step.  Each
// step's Q and dO rows (and lse, delta) are gathered straight into LDS with
// LDS DMA, NST steps in flight, so the gather latency is covered without
// holding staging registers.  Per (tile, chunk):
//   S = Q K^T, P = 2^{c S - lse2}, dP = dO V^T, dS = P (dP - delta),
//   dV += P^T dO, dK += dS^T Q.
// Slot partials are summed through LDS at the end; no atomics.  With TT equal
// to the tiles of one KV block, all waves share that block's chunk list, so no
// wave idles on chunks that only another block selected.
// Rows outside the sequence and columns past D are loaded from clamped
// addresses (finite data); the masks zero their P and dS, and the columns are
// never stored.
// ----------------------------------------------------------------------------
// dK/dV masks.  The membership rows (one per KV block of the WG's TT tiles)
// are small: with QW <= kBitsW words they are staged in LDS once, so the masks
// are built from LDS instead of one global round trip per chunk batch.
template <int TT>
__device__ bool fta_stage_kv_bits(const AttnArgs& a, int bh, int wk, int Tb, uint32_t (*sBits)[kBitsW]) {
    const int qw = a.QW;
    const bool bits_lds = qw <= kBitsW;
    if (bits_lds) {
        for (int i = threadIdx.x; i < TT * qw; i += blockDim.x) {
            const int t = i / qw, w = i - (i / qw) * qw;
            const int mt = (wk * TT + t) / Tb;
            sBits[t][w] = (mt < a.Mkv) ? a.sel[((int64_t)bh * a.Mkv + mt) * qw + w] : 0u;
        }
        __syncthreads();
    }
    return bits_lds;
}

// Column masks of the WG's TT key tiles over 32-query chunks [seg0, seg0 + segn)
// (tile t x chunk cl -> bits over the chunk's 32 queries), then the ascending
// list of chunks any tile needs.  Returns the list length.
template <int TT>
__device__ int fta_build_kv_masks(const AttnArgs& a, int bh, int wk, int Tb, int seg0, int segn, bool bits_lds,
                                  const uint32_t (*sBits)[kBitsW], uint32_t (*sMask)[kSegC], int* sList,
                                  int* s_tmp) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int NTHR = blockDim.x, NW = NTHR >> 6;
    const int qw = a.QW;
    // masks: tile t x chunk (seg0 + cl) -> bits over the chunk's 32 queries.
    // A chunk overlaps at most 33 q-blocks, i.e. two bitmap words per tile.
    for (int cl = tid; cl < segn; cl += NTHR) {
        const int pc = 32 * (seg0 + cl);
        const int qb_a = pc / a.g;
        const int qb_b = min((pc + 31) / a.g, a.QM - 1);
        const int w_a = qb_a >> 5, w_b = qb_b >> 5;
        uint32_t w0[TT], w1[TT];
#pragma unroll
        for (int t = 0; t < TT; ++t) {
            if (bits_lds) {
                w0[t] = sBits[t][w_a];
                w1[t] = (w_b > w_a) ? sBits[t][w_b] : 0u;
            } else {
                const int mt = (wk * TT + t) / Tb;
                const uint32_t* srow = a.sel + ((int64_t)bh * a.Mkv + min(mt, a.Mkv - 1)) * qw;
                w0[t] = (mt < a.Mkv) ? srow[w_a] : 0u;
                w1[t] = (mt < a.Mkv && w_b > w_a) ? srow[w_b] : 0u;
            }
        }
        const uint32_t valid = fta_range_bits(a.q_pad - pc, a.q_pad + a.N - pc);
#pragma unroll
        for (int t = 0; t < TT; ++t) {
            uint32_t bits = 0u;
            for (int qb = qb_a; qb <= qb_b; ++qb) {
                const uint32_t w = ((qb >> 5) == w_a) ? w0[t] : w1[t];
                if ((w >> (qb & 31)) & 1u) bits |= fta_range_bits(qb * a.g - pc, qb * a.g + a.g - pc);
            }
            sMask[t][cl] = bits & valid;
        }
    }
    __syncthreads();
    int U = 0;
    for (int base = 0; base < segn; base += NTHR) {
        const int cl = base + tid;
        int any = 0;
        if (cl < segn) {
#pragma unroll
            for (int t = 0; t < TT; ++t) any |= (sMask[t][cl] != 0u);
        }
        int x = any;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const int y = __shfl_up(x, off, 64);
            if (lane >= off) x += y;
        }
        if (lane == 63) s_tmp[wave] = x;
        __syncthreads();
        int wbase = 0, tot = 0;
#pragma unroll
        for (int w = 0; w < NW; ++w) {
            const int t = s_tmp[w];
            if (w < wave) wbase += t;
            tot += t;
        }
        if (any) sList[U + wbase + x - any] = cl;
        __syncthreads();
        U += tot;
    }
    return U;
}

template <int D, int TT, int CS>
struct DkvShape {
    static constexpr int NW = TT * CS;
    static constexpr int NTHR = NW * 64;
    static constexpr int QSEG = D / 8;
    static constexpr int TILE = 32 * QSEG;                       // 16-byte slots per 32-row tile
    static constexpr int LQ = (2 * CS * TILE + NTHR - 1) / NTHR;  // DMA instructions per wave per step
    static constexpr int L = LQ + 1;                              // + one for lse / delta
    static constexpr int LD_OFF = LQ * NW * 1024;                 // byte offset of lse / delta in a step
    static constexpr int STAGE_B = LD_OFF + NW * 256;
    static constexpr int FIXED_B = TT * kSegC * 4 + kSegC * 4 + TT * kBitsW * 4 + 64;
    static constexpr int NST_FIT = (150 * 1024 - FIXED_B) / STAGE_B;
    static constexpr int NST = NST_FIT > 4 ? 4 : NST_FIT;
    static_assert(NST >= 2, "two steps must fit in LDS");
    static_assert((NST - 2) * L < 64, "vmcnt range");
};

template <int DT, int D, int TT, int CS, bool GQA = false>
__global__ __launch_bounds__(TT * CS * 64, 1) void fta_sparse_dkv_kernel(AttnArgs a) {
    using E = Elem<DT>;
    using Sh = DkvShape<D, TT, CS>;
    constexpr int NW = Sh::NW, QSEG = Sh::QSEG, TILE = Sh::TILE, LQ = Sh::LQ, NST = Sh::NST;
    using SW = FtaSwz<QSEG>;
    constexpr int KS = D / 16;
    constexpr int DT32 = D / 32;
    static_assert(CS == 1 || TT * 32 * D * 4 <= NST * Sh::STAGE_B, "reduction tile must fit the staging buffers");
    __shared__ __align__(1024) unsigned char sStage[NST][Sh::STAGE_B];
    __shared__ uint32_t sMask[TT][kSegC];
    __shared__ int sList[kSegC];
    __shared__ uint32_t sBits[TT][kBitsW];
    __shared__ int s_tmp[8];

    const int wgi = fta_xcd_remap(blockIdx.x, a.total);
    const int bhk = wgi / a.wg_per_bh;  // (b, K/V head)
    const int wk = wgi - bhk * a.wg_per_bh;
    const int b = bhk / a.Hk, hk = bhk - (bhk / a.Hk) * a.Hk;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int hf = lane >> 5;
    const int tt = wave % TT, slot = wave / TT;
    const int Tb = (a.kvb + 31) >> 5;  // 32-key tiles per KV block

    // this wave's key tile
    const int G = wk * TT + tt;
    const int mblk = G / Tb;
    const int tin = G - (G / Tb) * Tb;
    const bool tile_live = mblk < a.Mkv;
    const int krel = 32 * tin + (lane & 31);  // key of this lane's column, relative to block start
    const int tk = mblk * a.kvb - a.kv_pad + krel;
    const bool kok = tile_live && krel < a.kvb && tk >= 0 && tk < a.N;

    const uint16_t* kp = a.k + b * a.k_sb + hk * a.k_sh;
    const uint16_t* vp = a.v + b * a.v_sb + hk * a.v_sh;
    // query-side operands of the query head being walked (set per head below)
    const uint16_t* qp = nullptr;
    const uint16_t* dp = nullptr;
    const float* lsep = nullptr;
    const float* dlp = nullptr;

    uint4 kf[KS], vf[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
        const int d = ks * 16 + hf * 8;
        const bool ok = kok && d < a.Dreal;
        kf[ks] = ok ? *reinterpret_cast<const uint4*>(kp + (int64_t)tk * a.k_sn + d) : fta_zero4();
        vf[ks] = ok ? *reinterpret_cast<const uint4*>(vp + (int64_t)tk * a.v_sn + d) : fta_zero4();
    }
    // complete the register loads here: the DMA steps below are invisible to the
    // compiler, which would otherwise wait for these loads (and with them every
    // DMA issued before their first use) inside the step loop
    fta_wait_vmcnt<0>();

    // Per-lane DMA sources.  Step layout: [Q slot 0..CS-1][dO slot 0..CS-1] 32-row
    // tiles, then lse / delta.  Instruction i of this wave fills 1 KB block
    // blk = i * NW + wave; a block never straddles a tile, so its tensor (ten)
    // and slot (sl) are wave-uniform, while the row and 16-byte slot are per
    // lane and the same for every step.  roff[i] = row * stride + column.
    int64_t roff[LQ];  // bytes
#pragma unroll
    for (int i = 0; i < LQ; ++i) {
        const int blk = i * NW + wave;
        const int ten = (blk * 64) / (CS * TILE);
        const int r2 = (blk * 64 + lane) % TILE;
        const int row = r2 / QSEG;
        int j = SW::slot(row, r2 - row * QSEG);
        if (j * 8 >= a.Dreal) j = 0;  // columns past D: any finite data (never stored)
        roff[i] = 2 * ((int64_t)row * (ten == 1 ? a.d_sn : a.q_sn) + j * 8);
    }
    // lse / delta lane: value v = wave * 64 + lane -> (which array, slot, row)
    const int lv = wave * 64 + lane;
    const bool l_isd = lv >= 32 * CS && lv < 64 * CS;
    const int l_sl = (lv < 64 * CS) ? ((lv >> 5) % CS) : 0;
    const int l_row = lv & 31;
    const float* l_base = nullptr;
    const uint32_t lds0 = fta_lds_addr(&sStage[0][0]);

    f32x16 dka[DT32], dva[DT32];
#pragma unroll
    for (int dt = 0; dt < DT32; ++dt)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            dka[dt][i] = 0.f;
            dva[dt][i] = 0.f;
        }

    // the query heads that share this K/V head (one without GQA): their
    // membership, Q, dO, lse and delta; dK / dV accumulate over all of them
    const int ngq = GQA ? a.G : 1;  // a constant 1 without GQA: no head loop in that code
    for (int gq = 0; gq < ngq; ++gq) {
        const int h = hk * a.G + gq;
        const int bh = b * a.H + h;
        qp = a.q + b * a.q_sb + h * a.q_sh;
        dp = a.dout + b * a.d_sb + h * a.d_sh;
        lsep = a.lse_in + (int64_t)bh * a.N;
        dlp = a.delta_in + (int64_t)bh * a.N;
        l_base = l_isd ? dlp : lsep;
        if (gq > 0) __syncthreads();  // the previous head's membership rows are no longer read
        const bool bits_lds = fta_stage_kv_bits<TT>(a, bh, wk, Tb, sBits);
        for (int seg0 = 0; seg0 < a.NC; seg0 += kSegC) {
            const int segn = min(kSegC, a.NC - seg0);
            const int U = fta_build_kv_masks<TT>(a, bh, wk, Tb, seg0, segn, bits_lds, sBits, sMask, sList, s_tmp);
            if (U == 0) continue;
            const int nsteps = (U + CS - 1) / CS;

            // gather step k (chunks k*CS .. k*CS + CS - 1 of the union list) into stage buffer st
            auto issue = [&](int st, int k) {
                const uint32_t sbase = lds0 + st * Sh::STAGE_B;
                const int u0 = k * CS;
                int cs[CS];
                bool inner = true;  // every row of every chunk lies in [0, N)
#pragma unroll
                for (int sl = 0; sl < CS; ++sl) {
                    cs[sl] = __builtin_amdgcn_readfirstlane(seg0 + sList[min(u0 + sl, U - 1)]);
                    const int t0 = 32 * cs[sl] - a.q_pad;
                    inner = inner && t0 >= 0 && t0 + 31 < a.N;
                }
                if (inner) {
#pragma unroll
                    for (int i = 0; i < LQ; ++i) {
                        const int blk = i * NW + wave;
                        const int ten = (blk * 64) / (CS * TILE);
                        const int sl = ((blk * 64) / TILE) % CS;
                        const int64_t t0 = 32 * cs[sl] - a.q_pad;
                        const char* base = reinterpret_cast<const char*>(ten == 1 ? dp + t0 * a.d_sn : qp + t0 * a.q_sn);
                        fta_dma16_at(base + roff[i], sbase + blk * 1024);
                    }
                } else {  // a chunk at a sequence edge: clamp its rows (masked off) into [0, N)
#pragma unroll
                    for (int i = 0; i < LQ; ++i) {
                        const int blk = i * NW + wave;
                        const int ten = (blk * 64) / (CS * TILE);
                        const int sl = ((blk * 64) / TILE) % CS;
                        const int r2 = (blk * 64 + lane) % TILE;
                        const int row = r2 / QSEG;
                        int j = SW::slot(row, r2 - row * QSEG);
                        if (j * 8 >= a.Dreal) j = 0;
                        const int t = min(max(32 * cs[sl] - a.q_pad + row, 0), a.N - 1);
                        fta_dma16_at((ten == 1 ? dp + (int64_t)t * a.d_sn : qp + (int64_t)t * a.q_sn) + j * 8,
                                     sbase + blk * 1024);
                    }
                }
                int c = cs[0];
#pragma unroll
                for (int sl = 1; sl < CS; ++sl) c = (l_sl == sl) ? cs[sl] : c;
                const int t = min(max(32 * c - a.q_pad + l_row, 0), a.N - 1);
                fta_dma4_at(l_base + t, sbase + Sh::LD_OFF + wave * 256);
            };

#pragma unroll
            for (int k = 0; k < NST - 1; ++k)
                if (k < nsteps) issue(k, k);
            int cur = 0;  // stage buffer of step k
            for (int k = 0; k < nsteps; ++k) {
                if (k + NST - 2 < nsteps)
                    fta_wait_vmcnt<Sh::L * (NST - 2)>();
                else
                    fta_wait_vmcnt<0>();
                __syncthreads();  // step k visible to all waves; step k - 1's buffer is free
                if (k + NST - 1 < nsteps) issue(cur == 0 ? NST - 1 : cur - 1, k + NST - 1);
                const int u = k * CS + slot;
                const uint32_t mk = (u < U) ? __builtin_amdgcn_readfirstlane(sMask[tt][sList[u]]) : 0u;
                if (mk) {
                    const uint16_t* qb = reinterpret_cast<const uint16_t*>(&sStage[cur][0]) + slot * TILE * 8;
                    const uint16_t* ob = qb + CS * TILE * 8;
                    const float* ld = reinterpret_cast<const float*>(&sStage[cur][Sh::LD_OFF]);
                    // Phased so that LDS latency overlaps MFMA work without exceeding the
                    // 256 VGPRs: (1) operand rows, (2) S and dP MFMAs, (3) transposed
                    // operands and lse / delta (while those MFMAs run), (4) softmax,
                    // (5) dV and dK MFMAs.  sched_barrier keeps the phases in order.
                    uint4 qa[KS], oa[KS];
#pragma unroll
                    for (int ks = 0; ks < KS; ++ks) {
                        const int off = SW::off(lane & 31, 2 * ks + hf);
                        qa[ks] = *reinterpret_cast<const uint4*>(qb + off);
                        oa[ks] = *reinterpret_cast<const uint4*>(ob + off);
                    }
                    f32x16 s, dpv;
#pragma unroll
                    for (int i = 0; i < 16; ++i) {
                        s[i] = 0.f;
                        dpv[i] = 0.f;
                    }
#pragma unroll
                    for (int ks = 0; ks < KS; ++ks) {
                        s = E::mma(qa[ks], kf[ks], s);
                        dpv = E::mma(oa[ks], vf[ks], dpv);
                    }
                    __builtin_amdgcn_sched_group_barrier(0x100, 2 * KS, 0);  // all operand-row reads
                    __builtin_amdgcn_sched_group_barrier(0x008, 2 * KS, 0);  // then the S / dP MFMAs
                    __builtin_amdgcn_sched_barrier(0);
                    uint4 to[2][DT32], tq[2][DT32];
#pragma unroll
                    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
                        for (int dt = 0; dt < DT32; ++dt) {
                            to[ks][dt] = fta_tr_frag_sw<QSEG>(ob, ks * 16, dt * 32, lane);
                            tq[ks][dt] = fta_tr_frag_sw<QSEG>(qb, ks * 16, dt * 32, lane);
                        }
                    float lr[16], dr[16];
#pragma unroll
                    for (int i = 0; i < 16; ++i) {
                        const int r = c_row(i, lane);
                        lr[i] = ld[slot * 32 + r];
                        dr[i] = ld[(CS + slot) * 32 + r];
                    }
                    __builtin_amdgcn_sched_barrier(0);
                    uint4 pf[2], dsf[2];
#pragma unroll
                    for (int ks = 0; ks < 2; ++ks) {
                        float pv[8], dv8[8];
#pragma unroll
                        for (int e = 0; e < 8; ++e) {
                            const int i = 8 * ks + e;
                            const int r = c_row(i, lane);
                            // a selected row with a valid key has a finite lse
                            const bool ok = kok && ((mk >> r) & 1u);
                            const float p = ok ? fta_exp2(fmaf(s[i], a.c, -lr[i] * 1.4426950408889634f)) : 0.f;
                            pv[e] = p;
                            dv8[e] = p * (dpv[i] - dr[i]);
                        }
                        pf[ks] = make_uint4(E::pack2(pv[0], pv[1]), E::pack2(pv[2], pv[3]), E::pack2(pv[4], pv[5]),
                                            E::pack2(pv[6], pv[7]));
                        dsf[ks] = make_uint4(E::pack2(dv8[0], dv8[1]), E::pack2(dv8[2], dv8[3]),
                                             E::pack2(dv8[4], dv8[5]), E::pack2(dv8[6], dv8[7]));
                    }
#pragma unroll
                    for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
                        for (int dt = 0; dt < DT32; ++dt) {
                            dva[dt] = E::mma(pf[ks], to[ks][dt], dva[dt]);
                            dka[dt] = E::mma(dsf[ks], tq[ks][dt], dka[dt]);
                        }
                    }
                }
                cur = (cur == NST - 1) ? 0 : cur + 1;
            }
            __syncthreads();  // all waves done with the stage buffers, sMask and sList
        }
    }

    if (CS > 1) {
        // sum the slot partials into slot 0, one slot and one operand at a time;
        // lane-linear layout [tile][dt][i][lane] keeps LDS accesses conflict-free
        float* red = reinterpret_cast<float*>(&sStage[0][0]);
#pragma unroll
        for (int sl = 1; sl < CS; ++sl) {
#pragma unroll
            for (int which = 0; which < 2; ++which) {
                if (slot == sl) {
#pragma unroll
                    for (int dt = 0; dt < DT32; ++dt)
#pragma unroll
                        for (int i = 0; i < 16; ++i)
                            red[((tt * DT32 + dt) * 16 + i) * 64 + lane] = which ? dva[dt][i] : dka[dt][i];
                }
                __syncthreads();
                if (slot == 0) {
#pragma unroll
                    for (int dt = 0; dt < DT32; ++dt)
#pragma unroll
                        for (int i = 0; i < 16; ++i) {
                            const float x = red[((tt * DT32 + dt) * 16 + i) * 64 + lane];
                            if (which)
                                dva[dt][i] += x;
                            else
                                dka[dt][i] += x;
                        }
                }
                __syncthreads();
            }
        }
    }

    if (!tile_live || slot != 0) return;
    // C layout: lane column = d (dt * 32 + lane & 31), rows = keys c_row(i, lane)
    uint16_t* kout = a.out0 + b * a.o0_sb + hk * a.o0_sh;
    uint16_t* vout = a.out1 + b * a.o1_sb + hk * a.o1_sh;
#pragma unroll
    for (int dt = 0; dt < DT32; ++dt) {
        const int d = dt * 32 + (lane & 31);
        if (d >= a.Dreal) continue;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int kr = 32 * tin + c_row(i, lane);
            const int t = mblk * a.kvb - a.kv_pad + kr;
            if (kr < a.kvb && t >= 0 && t < a.N) {
                const uint32_t pk = E::pack2(dka[dt][i] * a.scale, dva[dt][i]);
                kout[(int64_t)t * a.o0_sn + d] = (uint16_t)(pk & 0xffffu);
                vout[(int64_t)t * a.o1_sn + d] = (uint16_t)(pk >> 16);
            }
        }
    }
}

// ----------------------------------------------------------------------------
// dK / dV with the work of each key tile split over two waves (KV blocks of 33
// to 64 keys, D = 64, 128 or 256).  The WG owns the two 32-key tiles of one KV block;
// wave (tt, 0) holds K of tile tt and accumulates dV, wave (tt, 1) holds V of
// tile tt and accumulates dK, both over the full D.  Per chunk of 32 queries:
//   wave (tt, 0):  S = Q K^T,  P = 2^{c S - lse2}  -> LDS;  dV += P^T dO
//   wave (tt, 1):  dP = dO V^T;  (P from LDS)  dS = P (dP - delta);  dK += dS^T Q
// P crosses once, in fp32, so dS is formed from the same fp32 P as with one
// wave per tile.  Each wave evaluates only its own half of the elementwise work
// (the exponentials or the dS products), one of K / V and one set of
// accumulators, so a WG fits twice on a CU (registers <= 256 per lane, LDS <
// 80 KB): one WG's mask building and gather latency overlap the other's MFMAs.
// At D = 256 (twice the stage bytes and accumulators) one WG runs per CU, with
// the accumulators in the 512-register budget of one wave per SIMD.
// One chunk per step; NST steps of Q, dO, lse and delta in flight through LDS
// DMA, as in fta_sparse_dkv_kernel.
// ----------------------------------------------------------------------------
template <int D>
struct DkvSplitShape {
    static constexpr int NW = 4;
    static constexpr int NTHR = 256;
    static constexpr int QSEG = D / 8;
    static constexpr int TILE = 32 * QSEG;              // 16-byte slots per 32-row tile
    static constexpr int LQ = 2 * TILE / NTHR;          // DMA instructions per wave per step (Q, dO)
    static constexpr int L = LQ + 1;                    // + lse / delta (wave 0)
    static constexpr int LD_OFF = 2 * TILE * 16;        // byte offset of lse / delta in a step
    static constexpr int STAGE_B = LD_OFF + 256;
    static constexpr int NST = (D <= 64) ? 4 : 3;
    static constexpr int WPC = (D <= 128) ? 2 : 1;  // WGs per CU
    static_assert(2 * TILE % NTHR == 0, "whole DMA instructions per wave");
    static_assert(NST >= 3, "steps k - 1 and k live, at least one in flight");
    static_assert(NST * STAGE_B + 2 * 2 * 32 * 32 * 4 + 3 * kSegC * 4 + 2 * kBitsW * 4 + 64 <= 160 * 1024 / WPC,
                  "WPC WGs per CU");
};

template <int DT, int D, bool GQA, bool SPLIT>
__global__ __launch_bounds__(256, DkvSplitShape<D>::WPC) void fta_sparse_dkv_split_kernel(AttnArgs a) {
    using E = Elem<DT>;
    using Sh = DkvSplitShape<D>;
    constexpr int NW = Sh::NW, QSEG = Sh::QSEG, TILE = Sh::TILE, LQ = Sh::LQ, NST = Sh::NST;
    // the 8-row swizzle (V = 1): this kernel ran 2-3% faster with it than with the
    // conflict-free 16-row one, measured (C3 / C3-iid backward), despite its 2-way
    // conflicts on the 16-byte operand reads
    using SW = FtaSwz<QSEG, 1>;
    constexpr int KS = D / 16;
    constexpr int DT32 = D / 32;  // 32-column d tiles
    constexpr int TT = 2;
    __shared__ __align__(1024) unsigned char sStage[NST][Sh::STAGE_B];
    __shared__ float sX[2][TT][16][64];  // [step parity][tile][i][lane]: P of the last two steps
    __shared__ uint32_t sMask[TT][kSegC];
    __shared__ int sList[kSegC];
    __shared__ uint32_t sBits[TT][kBitsW];
    __shared__ int s_tmp[8];

    const int wgi = fta_xcd_remap(blockIdx.x, a.total);
    int hp, wk0, sp = 0;  // head position, launch rank, part
    if constexpr (SPLIT) {
        const int per = a.wg_per_bh * a.nsplit;
        hp = wgi / per;
        const int r = wgi - hp * per;
        wk0 = r / a.nsplit;
        sp = r - wk0 * a.nsplit;
    } else {
        hp = wgi / a.wg_per_bh;
        wk0 = wgi - hp * a.wg_per_bh;
    }
    const int bhk = a.head_perm ? a.head_perm[hp] : hp;  // (b, K/V head)
    const int wk = a.kv_order ? a.kv_order[(int64_t)bhk * a.wg_per_bh + wk0] : wk0;  // KV block
    const int b = bhk / a.Hk, hk = bhk - (bhk / a.Hk) * a.Hk;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int hf = lane >> 5;
    const int tt = wave & 1;
    const bool hv = (wave >> 1) != 0;  // wave-uniform role: false = K / P / dV, true = V / dS / dK
    const int Tb = 2;

    const int krel = 32 * tt + (lane & 31);  // key of this lane's column, relative to block start
    const int tk = wk * a.kvb - a.kv_pad + krel;
    const bool kok = krel < a.kvb && tk >= 0 && tk < a.N;

    // query-side operands of the query head being walked (set per head below)
    const uint16_t* qp = nullptr;
    const uint16_t* dp = nullptr;
    const float* lsep = nullptr;
    const float* dlp = nullptr;

    // K (role 0) or V (role 1) rows of this tile, full D
    uint4 kv[KS];
    {
        const uint16_t* src = hv ? a.v + b * a.v_sb + hk * a.v_sh : a.k + b * a.k_sb + hk * a.k_sh;
        const int64_t sn = hv ? a.v_sn : a.k_sn;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            const int d = ks * 16 + hf * 8;
            kv[ks] = (kok && d < a.Dreal) ? *reinterpret_cast<const uint4*>(src + (int64_t)tk * sn + d) : fta_zero4();
        }
    }
    // the first query head's membership rows (the staging waits for the K/V loads too)
    bool bits_lds = fta_stage_kv_bits<TT>(a, b * a.H + hk * a.G, wk, Tb, sBits);
    // complete the register loads: the DMAs below are invisible to the compiler
    fta_wait_vmcnt<0>();

    // Per-lane DMA sources (as in fta_sparse_dkv_kernel with one chunk slot):
    // instruction i of this wave fills 1 KB block blk = i * NW + wave of the
    // [Q tile][dO tile] step; roff[i] = row * stride + column, in bytes.
    int64_t roff[LQ];
#pragma unroll
    for (int i = 0; i < LQ; ++i) {
        const int blk = i * NW + wave;
        const int ten = (blk * 64) / TILE;
        const int r2 = (blk * 64 + lane) % TILE;
        const int row = r2 / QSEG;
        int j = SW::slot(row, r2 - row * QSEG);
        if (j * 8 >= a.Dreal) j = 0;  // columns past D: any finite data (never stored)
        roff[i] = 2 * ((int64_t)row * (ten == 1 ? a.d_sn : a.q_sn) + j * 8);
    }
    // lse / delta: wave 0's DMA writes [lse 32][delta 32] (256 bytes)
    const int lv = wave * 64 + lane;
    const bool l_isd = lv >= 32 && lv < 64;
    const float* l_base = nullptr;
    const int l_row = lv & 31;
    const uint32_t lds0 = fta_lds_addr(&sStage[0][0]);

    // the rest runs in one copy per role, so each keeps only its own values live
    auto run = [&](auto role) {
        constexpr bool HV = decltype(role)::value;
        f32x16 acc[DT32];  // dV (role 0) or dK / scale (role 1): rows = keys, lane column = d
#pragma unroll
        for (int dt = 0; dt < DT32; ++dt)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[dt][i] = 0.f;

        // the query heads that share this K/V head (one without GQA): their
        // membership, Q, dO, lse and delta; dK / dV accumulate over all of them
        const int ngq = GQA ? a.G : 1;  // a constant 1 without GQA: no head loop in that code
        for (int gq = 0; gq < ngq; ++gq) {
            const int h = hk * a.G + gq;
            const int bh = b * a.H + h;
            qp = a.q + b * a.q_sb + h * a.q_sh;
            dp = a.dout + b * a.d_sb + h * a.d_sh;
            lsep = a.lse2_in + (int64_t)bh * a.N;  // log2 units: no per-element scaling
            dlp = a.delta_in + (int64_t)bh * a.N;
            l_base = l_isd ? dlp : lsep;
            if (gq > 0) {
                __syncthreads();  // the previous head's membership rows are no longer read
                bits_lds = fta_stage_kv_bits<TT>(a, bh, wk, Tb, sBits);
            }
            for (int seg0 = 0; seg0 < a.NC; seg0 += kSegC) {
                const int segn = min(kSegC, a.NC - seg0);
                const int Ua = fta_build_kv_masks<TT>(a, bh, wk, Tb, seg0, segn, bits_lds, sBits, sMask, sList, s_tmp);
                // this part's chunk-list positions [u_lo, u_lo + U) (workgroup-uniform)
                int u_lo = 0, U = Ua;
                if constexpr (SPLIT) {
                    u_lo = (Ua * sp) / a.nsplit;
                    U = (Ua * (sp + 1)) / a.nsplit - u_lo;
                }
                // no wave reads sMask / sList below when the part is empty
                if (U == 0) continue;
                const int* lst = sList + u_lo;

                // gather chunk list entry k into stage buffer st
                auto issue = [&](int st, int k) {
                    const uint32_t sbase = lds0 + st * Sh::STAGE_B;
                    const int c = __builtin_amdgcn_readfirstlane(seg0 + lst[k]);
                    const int t0 = 32 * c - a.q_pad;
                    if (t0 >= 0 && t0 + 31 < a.N) {
#pragma unroll
                        for (int i = 0; i < LQ; ++i) {
                            const int blk = i * NW + wave;
                            const int ten = (blk * 64) / TILE;
                            const char* base =
                                reinterpret_cast<const char*>(ten == 1 ? dp + (int64_t)t0 * a.d_sn : qp + (int64_t)t0 * a.q_sn);
                            fta_dma16_at(base + roff[i], sbase + blk * 1024);
                        }
                    } else {  // a chunk at a sequence edge: clamp its rows (masked off) into [0, N)
#pragma unroll
                        for (int i = 0; i < LQ; ++i) {
                            const int blk = i * NW + wave;
                            const int ten = (blk * 64) / TILE;
                            const int r2 = (blk * 64 + lane) % TILE;
                            const int row = r2 / QSEG;
                            int j = SW::slot(row, r2 - row * QSEG);
                            if (j * 8 >= a.Dreal) j = 0;
                            const int t = min(max(t0 + row, 0), a.N - 1);
                            fta_dma16_at((ten == 1 ? dp + (int64_t)t * a.d_sn : qp + (int64_t)t * a.q_sn) + j * 8,
                                         sbase + blk * 1024);
                        }
                    }
                    if (wave == 0) {  // lse and delta of the chunk's 32 rows: one 256-byte DMA
                        const int t = min(max(t0 + l_row, 0), a.N - 1);
                        fta_dma4_at(l_base + t, sbase + Sh::LD_OFF);
                    }
                };

                // Software pipeline, one barrier per step: iteration k computes S_k / P_k
                // and dV_k (role 0) and dP_k (role 1); role 1 forms dS_{k-1} from P_{k-1}
                // (written to LDS in iteration k - 1) and adds dK_{k-1}, so the stage
                // buffers of steps k - 1 and k are live and NST - 2 steps are in flight.
#pragma unroll
                for (int k = 0; k < NST - 2; ++k)
                    if (k < U) issue(k, k);
                int cur = 0;       // stage buffer of step k
                bool pm = false;   // step k - 1 left its accumulation (dV or dK) to do
                f32x16 dpp;        // role 1: dP_{k-1}
                uint4 af[2];       // A operand of that accumulation: P_{k-1} (role 0) or dS_{k-1} (role 1)
                for (int k = 0; k <= U; ++k) {
                    if (k + NST - 3 >= U)
                        fta_wait_vmcnt<0>();
                    else if (wave == 0)  // wave 0 issues the lse / delta DMA as well
                        fta_wait_vmcnt<Sh::L * (NST - 3)>();
                    else
                        fta_wait_vmcnt<(Sh::L - 1) * (NST - 3)>();
                    // step k visible; step k - 2's buffer is free; P_{k-1} visible, sX[k & 1] free
                    __syncthreads();
                    if (k + NST - 2 < U) issue(cur >= 2 ? cur - 2 : cur + NST - 2, k + NST - 2);
                    const int prv = cur == 0 ? NST - 1 : cur - 1;  // stage buffer of step k - 1
                    const uint32_t mk = (k < U) ? __builtin_amdgcn_readfirstlane(sMask[tt][lst[k]]) : 0u;
                    const uint16_t* qb = reinterpret_cast<const uint16_t*>(&sStage[cur][0]);
                    const uint16_t* ob = qb + TILE * 8;
                    const float* ld = reinterpret_cast<const float*>(&sStage[cur][Sh::LD_OFF]);
                    // B operand of step k - 1's accumulation: dO^T (role 0, dV) or Q^T (role 1, dK)
                    const uint16_t* bb1 =
                        reinterpret_cast<const uint16_t*>(&sStage[pm ? prv : cur][0]) + (HV ? 0 : TILE * 8);
                    if (!pm) af[0] = af[1] = fta_zero4();
                    if (HV && pm) {  // dS_{k-1} = P_{k-1} (dP_{k-1} - delta)
                        const float* ld1 = reinterpret_cast<const float*>(&sStage[prv][Sh::LD_OFF]);
#pragma unroll
                        for (int ks = 0; ks < 2; ++ks) {
                            float dv8[8];
#pragma unroll
                            for (int e = 0; e < 8; ++e) {
                                const int i = 8 * ks + e;
                                dv8[e] = sX[(k + 1) & 1][tt][i][lane] * (dpp[i] - ld1[32 + c_row(i, lane)]);
                            }
                            af[ks] = make_uint4(E::pack2(dv8[0], dv8[1]), E::pack2(dv8[2], dv8[3]),
                                                E::pack2(dv8[4], dv8[5]), E::pack2(dv8[6], dv8[7]));
                        }
                    }
                    // S_k / dP_k (a dependent chain) interleaved with step k - 1's
                    // accumulation (independent MFMAs): the matrix pipe stays fed
                    f32x16 own;  // S_k then P_k (role 0) or dP_k (role 1)
                    const uint16_t* ab = HV ? ob : qb;
                    auto mmas = [&](auto with_s, auto with_acc) {
                        constexpr bool WS = decltype(with_s)::value, WA = decltype(with_acc)::value;
                        if (WS) {
#pragma unroll
                            for (int i = 0; i < 16; ++i) own[i] = 0.f;
                        }
                        // fragments of link j + 1 load while link j's MFMAs run
                        uint4 fs[2], fa2[2];
                        auto load = [&](int j, int slot) {
                            if (WS) fs[slot] = *reinterpret_cast<const uint4*>(ab + SW::off(lane & 31, 2 * j + hf));
                            if (WA) fa2[slot] = fta_tr_frag_sw<QSEG, 1>(bb1, (j / DT32) * 16, (j % DT32) * 32, lane);
                        };
                        constexpr int NR = (WS ? 1 : 0) + (WA ? 2 : 0);  // LDS reads per link
                        constexpr int NM = (WS ? 1 : 0) + (WA ? 1 : 0);  // MFMAs per link
                        load(0, 0);
#pragma unroll
                        for (int j = 0; j < KS; ++j) {  // KS = 2 * DT32: one accumulation MFMA per chain link
                            if (j + 1 < KS) load(j + 1, (j + 1) & 1);
                            if (WS) own = E::mma(fs[j & 1], kv[j], own);
                            if (WA) acc[j % DT32] = E::mma(af[j / DT32], fa2[j & 1], acc[j % DT32]);
                        }
                        __builtin_amdgcn_sched_group_barrier(0x100, NR, 0);
#pragma unroll
                        for (int j = 0; j < KS; ++j) {
                            if (j + 1 < KS) __builtin_amdgcn_sched_group_barrier(0x100, NR, 0);
                            __builtin_amdgcn_sched_group_barrier(0x008, NM, 0);
                        }
                    };
                    // One instruction stream for every case (separate variants cost the
                    // register budget): without a pending accumulation the A operand is zero
                    // and the B operand the current step's finite data (acc += 0 exactly);
                    // without a chain the S / dP result is discarded.
                    if (mk || pm) mmas(std::true_type{}, std::true_type{});
                    if (mk) {
                        if (!HV) {  // P_k = 2^{c S_k - lse2}: to LDS for role 1, packed for dV_k
                            if (mk == 0xffffffffu && __ballot(!kok) == 0ull) {
                                // every row of the chunk selected, every key valid: no mask
#pragma unroll
                                for (int i = 0; i < 16; ++i) own[i] = fta_exp2(fmaf(own[i], a.c, -ld[c_row(i, lane)]));
                            } else {
#pragma unroll
                                for (int i = 0; i < 16; ++i) {
                                    const int r = c_row(i, lane);
                                    // a selected row with a valid key has a finite lse
                                    const bool ok = kok && ((mk >> r) & 1u);
                                    const float ex = fta_exp2(fmaf(own[i], a.c, -ld[r]));
                                    own[i] = ok ? ex : 0.f;
                                }
                            }
#pragma unroll
                            for (int i = 0; i < 16; ++i) sX[k & 1][tt][i][lane] = own[i];
#pragma unroll
                            for (int ks = 0; ks < 2; ++ks)
                                af[ks] = make_uint4(E::pack2(own[8 * ks], own[8 * ks + 1]),
                                                    E::pack2(own[8 * ks + 2], own[8 * ks + 3]),
                                                    E::pack2(own[8 * ks + 4], own[8 * ks + 5]),
                                                    E::pack2(own[8 * ks + 6], own[8 * ks + 7]));
                        } else {
                            dpp = own;
                        }
                    }
                    pm = mk != 0u;
                    cur = (cur == NST - 1) ? 0 : cur + 1;
                }
                __syncthreads();  // all waves done with the stage buffers, sMask and sList
            }
        }

        // C layout: lane column = d, rows = keys c_row(i, lane); role 0 stores dV, role 1 dK
        if constexpr (SPLIT) {
            // the part's unscaled fp32 dK (role 1) or dV (role 0), rows wk * 64 + key
            float* po = a.part_o + ((((int64_t)(HV ? 0 : 1) * a.nsplit + sp) * a.nbh + bhk) * a.npq +
                                    (int64_t)wk * 64 + 32 * tt) * D;
#pragma unroll
            for (int dt = 0; dt < DT32; ++dt)
#pragma unroll
                for (int i = 0; i < 16; ++i) po[(int64_t)c_row(i, lane) * D + dt * 32 + (lane & 31)] = acc[dt][i];
            return;
        }
        uint16_t* out = HV ? a.out0 + b * a.o0_sb + hk * a.o0_sh : a.out1 + b * a.o1_sb + hk * a.o1_sh;
        const int64_t osn = HV ? a.o0_sn : a.o1_sn;
        const float osc = HV ? a.scale : 1.f;
#pragma unroll
        for (int dt = 0; dt < DT32; ++dt) {
            const int d = dt * 32 + (lane & 31);
            if (d >= a.Dreal) continue;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int kr = 32 * tt + c_row(i, lane);
                const int t = wk * a.kvb - a.kv_pad + kr;
                if (kr < a.kvb && t >= 0 && t < a.N) out[(int64_t)t * osn + d] = (uint16_t)(E::pack2(acc[dt][i] * osc, 0.f) & 0xffffu);
            }
        }
    };
    if (hv)
        run(std::true_type{});
    else
        run(std::false_type{});
}


// Sum of the split dK/dV parts: one thread per (b·K/V head, key, 8 columns) and
// tensor; dK = scale · sum_p dK_p, dV = sum_p dV_p, parts added in order.
template <int DT, int D>
__global__ __launch_bounds__(256) void fta_dkv_combine_kernel(AttnArgs a) {
    using E = Elem<DT>;
    constexpr int DC = D / 8;
    const int64_t per = (int64_t)a.nbh * a.N * DC;
    int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= 2 * per) return;
    const int ten = idx >= per;  // 0: dK, 1: dV
    idx -= ten * per;
    const int dc = (int)(idx % DC);
    const int64_t rest = idx / DC;
    const int t = (int)(rest % a.N), bhk = (int)(rest / a.N);
    const int d0 = dc * 8;
    if (d0 >= a.Dreal) return;
    const int kp = t + a.kv_pad;
    const int64_t row = (int64_t)(kp / a.kvb) * 64 + kp % a.kvb;
    float o[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int sp = 0; sp < a.nsplit; ++sp) {
        const float* src = a.part_o + ((((int64_t)ten * a.nsplit + sp) * a.nbh + bhk) * a.npq + row) * D + d0;
        const float4 x0 = *reinterpret_cast<const float4*>(src);
        const float4 x1 = *reinterpret_cast<const float4*>(src + 4);
        o[0] += x0.x;
        o[1] += x0.y;
        o[2] += x0.z;
        o[3] += x0.w;
        o[4] += x1.x;
        o[5] += x1.y;
        o[6] += x1.z;
        o[7] += x1.w;
    }
    const float sc = ten ? 1.f : a.scale;
    const int b = bhk / a.Hk, hk = bhk - (bhk / a.Hk) * a.Hk;
    uint16_t* op = ten ? a.out1 + b * a.o1_sb + hk * a.o1_sh + (int64_t)t * a.o1_sn + d0
                       : a.out0 + b * a.o0_sb + hk * a.o0_sh + (int64_t)t * a.o0_sn + d0;
    *reinterpret_cast<uint2*>(op) = make_uint2(E::pack2(o[0] * sc, o[1] * sc), E::pack2(o[2] * sc, o[3] * sc));
    *reinterpret_cast<uint2*>(op + 4) = make_uint2(E::pack2(o[4] * sc, o[5] * sc), E::pack2(o[6] * sc, o[7] * sc));
}

// lse2 = lse * log2(e) (the same fp32 product the kernels formed per element)
__global__ __launch_bounds__(256) void fta_lse2_kernel(const float* __restrict__ lse, float* __restrict__ lse2,
                                                       int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) lse2[i] = lse[i] * 1.4426950408889634f;
}

// ----------------------------------------------------------------------------
// Host side
// ----------------------------------------------------------------------------
namespace {

struct Geo {
    int Dk, Mkv, QM, nch, sbk, Npk, NC, Npq;
};

int geometry(int B, int H, int N, int D, int g, int kvb, int qph, int qpt, int kvph, int kvpt, int QM, Geo* o) {
    if (B <= 0 || H <= 0 || N <= 0 || D <= 0) return fta::arg_error("sparse_attn: dims must be positive");
    if (D % 16 != 0) return fta::arg_error("sparse_attn: D must be a positive multiple of 16");
    if (D > 256) return fta::arg_error("sparse_attn: D must be <= 256");
    if (g <= 0) return fta::arg_error("sparse_attn: q_block_size must be positive");
    if (kvb <= 0) return fta::arg_error("sparse_attn: kv_block_size must be positive");
    if (qph < 0 || qpt < 0 || qph >= g || qpt >= g) return fta::arg_error("sparse_attn: bad q_padding");
    if (kvph < 0 || kvpt < 0 || kvph >= kvb || kvpt >= kvb) return fta::arg_error("sparse_attn: bad kv_padding");
    const int64_t nq = (int64_t)qph + N + qpt, nk = (int64_t)kvph + N + kvpt;
    if (nq % g) return fta::arg_error("sparse_attn: q_pad_head + N + q_pad_tail must be divisible by q_block_size");
    if (nk % kvb) return fta::arg_error("sparse_attn: kv_pad_head + N + kv_pad_tail must be divisible by kv_block_size");
    if (nq / g != QM) return fta::arg_error("sparse_attn: merged_indices dim 2 must equal QM");
    // D <= 128 runs on the 64- or 128-column kernels (columns past D meet zero
    // Q / dO columns and are never stored)
    o->Dk = (D <= 64) ? 64 : (D <= 128) ? 128 : fta::kernel_head_dim(D);
    o->Mkv = (int)(nk / kvb);
    o->QM = QM;
    o->nch = (kvb + 63) / 64;
    o->sbk = o->nch * 64;
    o->Npk = o->Mkv * o->sbk;
    o->NC = (int)((nq + 31) / 32);
    o->Npq = o->NC * 32;
    return FTA_OK;
}

void fill_common(AttnArgs& a, int H, int N, int D, int g, int kvb, int qph, int kvph, float scale, const Geo& G) {
    a.H = H;
    a.Hk = H;  // no GQA unless the caller sets Hk / G
    a.G = 1;
    a.N = N;
    a.Dreal = D;
    a.g = g;
    a.kvb = kvb;
    a.q_pad = qph;
    a.kv_pad = kvph;
    a.Mkv = G.Mkv;
    a.NC = G.NC;
    a.QM = G.QM;
    a.QW = (G.QM + 31) / 32;
    a.scale = scale;
    a.c = scale * 1.4426950408889634f;
}

template <int DT>
int launch_fwd_dt(AttnArgs& a, int Dk, int grid, hipStream_t st) {
    // the pipelined kernel keeps per-lane row offsets (64 rows x stride) in 32 bits
    const bool pipe_ok = a.k_sn <= (1 << 24) && a.v_sn <= (1 << 24);
    switch (Dk) {
#define FTA_FWD(DK, TPW, NW)                                                                              \
    case DK:                                                                                              \
        hipLaunchKernelGGL((fta_sparse_fwd_kernel<DT, DK, TPW, NW>), dim3(grid), dim3(NW * 64), 0, st, a); \
        break;
        FTA_FWD(32, 1, 8)
        case 64:
            if (pipe_ok && a.nsplit > 1)
                hipLaunchKernelGGL((fta_sparse_fwd_pipe_kernel<DT, 64, 8, true>), dim3(grid), dim3(512), 0, st, a);
            else if (pipe_ok)
                hipLaunchKernelGGL((fta_sparse_fwd_pipe_kernel<DT, 64, 8, false>), dim3(grid), dim3(512), 0, st, a);
            else
                hipLaunchKernelGGL((fta_sparse_fwd_kernel<DT, 64, 1, 8>), dim3(grid), dim3(512), 0, st, a);
            break;
        FTA_FWD(96, 1, 8)
        case 128:
            if (pipe_ok && a.nsplit > 1)
                hipLaunchKernelGGL((fta_sparse_fwd_pipe_kernel<DT, 128, 8, true>), dim3(grid), dim3(512), 0, st, a);
            else if (pipe_ok)
                hipLaunchKernelGGL((fta_sparse_fwd_pipe_kernel<DT, 128, 8, false>), dim3(grid), dim3(512), 0, st, a);
            else
                hipLaunchKernelGGL((fta_sparse_fwd_kernel<DT, 128, 1, 8>), dim3(grid), dim3(512), 0, st, a);
            break;
        FTA_FWD(160, 1, 8)
        FTA_FWD(256, 1, 4)
#undef FTA_FWD
        default:
            return fta::arg_error("sparse_attn: unsupported head dim");
    }
    int rc = fta::check_launch("fta_sparse_fwd_kernel");
    if (rc != FTA_OK || !(pipe_ok && a.nsplit > 1)) return rc;
    const int64_t threads = (int64_t)a.nbh * a.N * (Dk / 8);
    const unsigned blocks = (unsigned)((threads + 255) / 256);
    if (Dk == 64)
        hipLaunchKernelGGL((fta_fwd_combine_kernel<DT, 64>), dim3(blocks), dim3(256), 0, st, a);
    else
        hipLaunchKernelGGL((fta_fwd_combine_kernel<DT, 128>), dim3(blocks), dim3(256), 0, st, a);
    return fta::check_launch("fta_fwd_combine_kernel");
}

template <int DT>
int launch_dq_dt(AttnArgs& a, int Dk, int grid, hipStream_t st) {
    // the pipelined kernel keeps per-lane row offsets (64 rows x stride) in 32 bits
    const bool pipe_ok = a.k_sn <= (1 << 24) && a.v_sn <= (1 << 24);
    // split walks (decided by the caller, grid included): the pipelined kernels (D 64 /
    // 128) or the register-staged ones (D 160 / 256)
    const bool split = a.nsplit > 1;
    if (split && !(Dk == 160 || Dk == 256 || ((Dk == 64 || Dk == 128) && pipe_ok)))
        return fta::arg_error("sparse_attn_bwd: no split dQ kernel for this shape");
    switch (Dk) {
#define FTA_DQ(DK, NW)                                                                                  \
    case DK:                                                                                             \
        if (split)                                                                                       \
            hipLaunchKernelGGL((fta_sparse_dq_kernel<DT, DK, NW, true>), dim3(grid), dim3(NW * 64), 0, st, a); \
        else                                                                                             \
            hipLaunchKernelGGL((fta_sparse_dq_kernel<DT, DK, NW, false>), dim3(grid), dim3(NW * 64), 0, st, a); \
        break;
        case 32:
            hipLaunchKernelGGL((fta_sparse_dq_kernel<DT, 32, 8, false>), dim3(grid), dim3(512), 0, st, a);
            break;
        case 64:
            if (split)
                hipLaunchKernelGGL((fta_sparse_dq_pipe_kernel<DT, 64, true>), dim3(grid), dim3(512), 0, st, a);
            else if (pipe_ok)
                hipLaunchKernelGGL((fta_sparse_dq_pipe_kernel<DT, 64, false>), dim3(grid), dim3(512), 0, st, a);
            else
                hipLaunchKernelGGL((fta_sparse_dq_kernel<DT, 64, 8, false>), dim3(grid), dim3(512), 0, st, a);
            break;
        case 96:
            hipLaunchKernelGGL((fta_sparse_dq_kernel<DT, 96, 8, false>), dim3(grid), dim3(512), 0, st, a);
            break;
        case 128:
            if (split)
                hipLaunchKernelGGL((fta_sparse_dq_pipe_kernel<DT, 128, true>), dim3(grid), dim3(512), 0, st, a);
            else if (pipe_ok)
                hipLaunchKernelGGL((fta_sparse_dq_pipe_kernel<DT, 128, false>), dim3(grid), dim3(512), 0, st, a);
            else
                hipLaunchKernelGGL((fta_sparse_dq_kernel<DT, 128, 8, false>), dim3(grid), dim3(512), 0, st, a);
            break;
        FTA_DQ(160, 4)
        FTA_DQ(256, 4)
#undef FTA_DQ
        default:
            return fta::arg_error("sparse_attn_bwd: unsupported head dim");
    }
    int rc = fta::check_launch("fta_sparse_dq_kernel");
    if (rc != FTA_OK || !split) return rc;
    const int64_t threads = (int64_t)a.nbh * a.N * (Dk / 8);
    const unsigned blocks = (unsigned)((threads + 255) / 256);
    switch (Dk) {
        case 64: hipLaunchKernelGGL((fta_dq_combine_kernel<DT, 64>), dim3(blocks), dim3(256), 0, st, a); break;
        case 128: hipLaunchKernelGGL((fta_dq_combine_kernel<DT, 128>), dim3(blocks), dim3(256), 0, st, a); break;
        case 160: hipLaunchKernelGGL((fta_dq_combine_kernel<DT, 160>), dim3(blocks), dim3(256), 0, st, a); break;
        default: hipLaunchKernelGGL((fta_dq_combine_kernel<DT, 256>), dim3(blocks), dim3(256), 0, st, a); break;
    }
    return fta::check_launch("fta_dq_combine_kernel");
}

// dK/dV launch shape: TT key tiles x CS chunk slots.  TT covers the 32-key tiles
// of one KV block when a block has at most two, so every wave of a workgroup
// shares one chunk list; longer blocks, and D = 256 (whose slot partials would
// spill), use one slot (TT = all waves).
template <int DT>
int launch_dkv_dt(AttnArgs& a, int Dk, int Tb, int B, int H, int ntiles, hipStream_t st) {
    const bool gqa = a.G > 1;
    // ns: parts per KV block (the split kernel with a.nsplit > 1), else 1
    auto go = [&](auto kern, int tt, int nw, int ns) {
        a.wg_per_bh = (ntiles + tt - 1) / tt;
        a.total = a.wg_per_bh * B * H * ns;
        hipLaunchKernelGGL(kern, dim3(a.total), dim3(nw * 64), 0, st, a);
    };
    switch (Dk) {
#define FTA_DKV_GO(DK, TTX, CSX)                                                             \
    (gqa ? go(fta_sparse_dkv_kernel<DT, DK, TTX, CSX, true>, TTX, TTX * CSX, 1)              \
         : go(fta_sparse_dkv_kernel<DT, DK, TTX, CSX, false>, TTX, TTX * CSX, 1))
#define FTA_DKV(DK, NW, TT1, CS1, TT2, CS2)                                                  \
    case DK:                                                                                 \
        if (Tb == 1)                                                                         \
            FTA_DKV_GO(DK, TT1, CS1);                                                        \
        else if (Tb == 2)                                                                    \
            FTA_DKV_GO(DK, TT2, CS2);                                                        \
        else                                                                                 \
            FTA_DKV_GO(DK, NW, 1);                                                           \
        break;
#define FTA_DKV_SPLIT(DK)                                                                            \
    if (a.nsplit > 1)                                                                                \
        gqa ? go(fta_sparse_dkv_split_kernel<DT, DK, true, true>, 2, 4, a.nsplit)                    \
            : go(fta_sparse_dkv_split_kernel<DT, DK, false, true>, 2, 4, a.nsplit);                  \
    else                                                                                             \
        gqa ? go(fta_sparse_dkv_split_kernel<DT, DK, true, false>, 2, 4, 1)                          \
            : go(fta_sparse_dkv_split_kernel<DT, DK, false, false>, 2, 4, 1)
        FTA_DKV(32, 8, 1, 4, 2, 4)
        case 64:
            if (Tb == 2)
                FTA_DKV_SPLIT(64);
            else if (Tb == 1)
                FTA_DKV_GO(64, 1, 4);
            else
                FTA_DKV_GO(64, 8, 1);
            break;
        FTA_DKV(96, 4, 1, 4, 2, 2)
        case 128:
            if (Tb == 2)
                FTA_DKV_SPLIT(128);
            else if (Tb == 1)
                FTA_DKV_GO(128, 1, 4);
            else
                FTA_DKV_GO(128, 4, 1);
            break;
        FTA_DKV(160, 4, 2, 2, 2, 2)
        case 256:
            if (Tb == 2)
                FTA_DKV_SPLIT(256);
            else
                FTA_DKV_GO(256, 4, 1);
            break;
#undef FTA_DKV_SPLIT
#undef FTA_DKV
#undef FTA_DKV_GO
        default:
            return fta::arg_error("sparse_attn_bwd: unsupported head dim");
    }
    int rc = fta::check_launch("fta_sparse_dkv_kernel");
    if (rc != FTA_OK || a.nsplit <= 1) return rc;
    // the parts' sums: dK and dV, one thread per (b * Hk, key, 8 columns) each
    const int64_t threads = 2 * (int64_t)a.nbh * a.N * (Dk / 8);
    const unsigned blocks = (unsigned)((threads + 255) / 256);
    if (Dk == 64)
        hipLaunchKernelGGL((fta_dkv_combine_kernel<DT, 64>), dim3(blocks), dim3(256), 0, st, a);
    else if (Dk == 128)
        hipLaunchKernelGGL((fta_dkv_combine_kernel<DT, 128>), dim3(blocks), dim3(256), 0, st, a);
    else
        hipLaunchKernelGGL((fta_dkv_combine_kernel<DT, 256>), dim3(blocks), dim3(256), 0, st, a);
    return fta::check_launch("fta_dkv_combine_kernel");
}

size_t sel_bytes(int B, int H, const Geo& G) {
    return fta::align_up((size_t)B * H * G.Mkv * ((G.QM + 31) / 32) * sizeof(uint32_t));
}

// the forward workspace: per-head work, head placement (fta_head_balance_kernel)
// and the 64 partial counts per head they are summed from
size_t fwd_bytes(int B, int H) { return fta::align_up((size_t)B * H * (2 + 64) * sizeof(int32_t)); }

// Forward parts per workgroup.  A grid of fewer than 128 workgroups (under half
// the CUs) is bound by each workgroup's sequential union walk, not by the chip:
// the pipelined kernel then splits every walk into up to 4 parts (256 / grid)
// and fta_fwd_combine_kernel merges them.
int fwd_nsplit(int B, int H, const Geo& G) {
    if (!(G.Dk == 64 || G.Dk == 128) || G.Mkv < 8) return 1;
    const int64_t wgs = (int64_t)((G.Npq + 255) / 256) * B * H;
    if (wgs >= 128) return 1;
    const int64_t ns = 256 / wgs;
    return (int)(ns > 4 ? 4 : ns < 2 ? 2 : ns);
}
// the parts' (m, L) and unnormalised O, after fwd_bytes in the workspace
size_t split_bytes(int B, int H, const Geo& G, int ns) {
    if (ns <= 1) return 0;
    const size_t rows = (size_t)ns * B * H * G.Npq;
    return fta::align_up(rows * sizeof(float2)) + fta::align_up(rows * G.Dk * sizeof(float));
}

// dQ's split walks on small grids: the forward's rule for the pipelined kernels
// (D 64 / 128, 256-query workgroups); the register-staged ones at D 160 / 256
// (128-query workgroups, one per CU) split while at most half the CUs are busy
int dq_nsplit(int B, int H, const Geo& G) {
    if (G.Dk == 64 || G.Dk == 128) return fwd_nsplit(B, H, G);
    if (!(G.Dk == 160 || G.Dk == 256) || G.Mkv < 8) return 1;
    const int64_t wgs = (int64_t)((G.Npq + 127) / 128) * B * H;
    if (wgs > 128) return 1;
    const int64_t ns = 256 / wgs;
    return (int)(ns > 4 ? 4 : ns < 2 ? 2 : ns);
}
// dQ's split parts, after bwd_bytes in the workspace of the combined backward
size_t dq_split_bytes(int B, int H, const Geo& G, int ns) {
    if (ns <= 1) return 0;
    return fta::align_up((size_t)ns * B * H * G.Npq * G.Dk * sizeof(float));
}

// dK/dV parts of the split kernel (64-key blocks, D 64 / 128 / 256) on small
// grids: fewer workgroups than the CUs hold (two per CU, one at D = 256) get
// up to 4 parts per KV block; [dK, dV][part][b * Hk][KV block * 64 + key][Dk]
// fp32, after bwd_bytes (dQ's parts reuse the same bytes after dK/dV is done)
int dkv_nsplit(int B, int Hk, int kv_block_size, const Geo& G) {
    if (!(kv_block_size > 32 && kv_block_size <= 64 && (G.Dk == 64 || G.Dk == 128 || G.Dk == 256))) return 1;
    const int64_t wgs = (int64_t)G.Mkv * B * Hk;
    const int64_t cap = (G.Dk <= 128) ? 512 : 256;
    if (wgs >= cap) return 1;
    const int64_t ns = cap / wgs;
    return (int)(ns > 4 ? 4 : ns < 2 ? 2 : ns);
}
size_t dkv_split_bytes(int B, int Hk, const Geo& G, int ns) {
    if (ns <= 1) return 0;
    return fta::align_up((size_t)2 * ns * B * Hk * G.Mkv * 64 * G.Dk * sizeof(float));
}

// the backward workspace: membership bitmap, lse in log2 units, dK/dV launch order (KV blocks, then heads)
size_t bwd_bytes(int B, int H, int N, const Geo& G) {
    return sel_bytes(B, H, G) + fta::align_up((size_t)B * H * N * sizeof(float)) +
           fta::align_up((size_t)B * H * G.Mkv * sizeof(int32_t)) + fta::align_up((size_t)B * H * 2 * sizeof(int32_t));
}

}  // namespace

extern "C" {

size_t fta_sparse_attn_fwd_workspace_size(int B, int H, int N, int D, int q_block_size, int kv_block_size,
                                          int q_pad_head, int q_pad_tail, int kv_pad_head, int kv_pad_tail) {
    Geo G;
    const int64_t nq = (int64_t)q_pad_head + N + q_pad_tail;
    const int QM = q_block_size > 0 ? (int)(nq / q_block_size) : 0;
    if (geometry(B, H, N, D, q_block_size, kv_block_size, q_pad_head, q_pad_tail, kv_pad_head, kv_pad_tail, QM,
                 &G) != FTA_OK)
        return 0;
    // per-head work and XCD placement of the heads, then the split parts
    return fwd_bytes(B, H) + split_bytes(B, H, G, fwd_nsplit(B, H, G));
}

int fta_sparse_attn_fwd_splits(int B, int H, int N, int D, int q_block_size, int kv_block_size, int q_pad_head,
                               int q_pad_tail, int kv_pad_head, int kv_pad_tail) {
    Geo G;
    const int64_t nq = (int64_t)q_pad_head + N + q_pad_tail;
    const int QM = q_block_size > 0 ? (int)(nq / q_block_size) : 0;
    if (geometry(B, H, N, D, q_block_size, kv_block_size, q_pad_head, q_pad_tail, kv_pad_head, kv_pad_tail, QM,
                 &G) != FTA_OK)
        return 0;
    return fwd_nsplit(B, H, G);
}

int fta_sparse_attn_fwd_gqa(const void* q, const int64_t* q_strides, const void* k, const int64_t* k_strides,
                            const void* v, const int64_t* v_strides, int dtype, int B, int H, int Hk, int N, int D,
                            const int32_t* merged_indices, int QM, int W, int q_block_size, int kv_block_size,
                            int q_pad_head, int q_pad_tail, int kv_pad_head, int kv_pad_tail, float scale,
                            void* o, const int64_t* o_strides, float* lse, void* workspace, size_t workspace_bytes,
                            void* stream) {
    FTA_TRY_BEGIN
    if (Hk <= 0 || H % Hk != 0) return fta::arg_error("sparse_attn: num_heads must be a multiple of num_kv_heads");
    Geo G;
    int rc = geometry(B, H, N, D, q_block_size, kv_block_size, q_pad_head, q_pad_tail, kv_pad_head, kv_pad_tail, QM,
                      &G);
    if (rc != FTA_OK) return rc;
    if (W <= 0) return fta::arg_error("sparse_attn: qblock_topk must be positive");
    hipStream_t st = (hipStream_t)stream;
    AttnArgs a = {};
    const int T = (G.Dk <= 160) ? 8 : 4;  // query tiles per workgroup
    const int64_t wgs = (int64_t)((G.Npq + 32 * T - 1) / (32 * T)) * B * H;
    // XCD placement of the heads by their work (only with a workspace: callers
    // that pass none keep the natural order; and only when the workgroups do not
    // all run at once, one per CU, where the placement cannot change the time)
    if (workspace != nullptr && workspace_bytes >= fwd_bytes(B, H) && wgs > 256) {
        int32_t* head_work = (int32_t*)workspace;
        int32_t* head_perm = head_work + B * H;
        if ((rc = fta::launch_head_order_merged(merged_indices, B * H, QM, W, G.Mkv, max(1, 256 / q_block_size), head_work, head_perm, st)) !=
            FTA_OK)
            return rc;
        a.head_perm = head_perm;
    }
    a.q = (const uint16_t*)q;
    a.q_sb = q_strides[0];
    a.q_sh = q_strides[1];
    a.q_sn = q_strides[2];
    a.k = (const uint16_t*)k;
    a.k_sb = k_strides[0];
    a.k_sh = k_strides[1];
    a.k_sn = k_strides[2];
    a.v = (const uint16_t*)v;
    a.v_sb = v_strides[0];
    a.v_sh = v_strides[1];
    a.v_sn = v_strides[2];
    a.merged = merged_indices;
    a.W = W;
    a.out0 = (uint16_t*)o;
    a.o0_sb = o_strides[0];
    a.o0_sh = o_strides[1];
    a.o0_sn = o_strides[2];
    a.lse = lse;
    fill_common(a, H, N, D, q_block_size, kv_block_size, q_pad_head, kv_pad_head, scale, G);
    a.Hk = Hk;
    a.G = H / Hk;
    a.wg_per_bh = (G.Npq + 32 * T - 1) / (32 * T);
    // split walks (small grids, pipelined kernel, workspace for the parts)
    const int ns = fwd_nsplit(B, H, G);
    const bool split = ns > 1 && workspace != nullptr &&
                       workspace_bytes >= fwd_bytes(B, H) + split_bytes(B, H, G, ns) && k_strides[2] <= (1 << 24) &&
                       v_strides[2] <= (1 << 24);
    a.nsplit = split ? ns : 1;
    a.nbh = B * H;
    a.npq = G.Npq;
    if (split) {
        const size_t rows = (size_t)ns * B * H * G.Npq;
        a.part_ml = (float2*)((char*)workspace + fwd_bytes(B, H));
        a.part_o = (float*)((char*)a.part_ml + fta::align_up(rows * sizeof(float2)));
    }
    a.total = a.wg_per_bh * B * H * a.nsplit;
    if (dtype == FTA_DTYPE_BF16) return launch_fwd_dt<FTA_DTYPE_BF16>(a, G.Dk, a.total, st);
    if (dtype == FTA_DTYPE_F16) return launch_fwd_dt<FTA_DTYPE_F16>(a, G.Dk, a.total, st);
    return fta::arg_error("sparse_attn: dtype must be bf16 or fp16");
    FTA_TRY_END
}

size_t fta_sparse_attn_bwd_workspace_size(int B, int H, int N, int D, int q_block_size, int kv_block_size,
                                          int q_pad_head, int q_pad_tail, int kv_pad_head, int kv_pad_tail) {
    Geo G;
    const int64_t nq = (int64_t)q_pad_head + N + q_pad_tail;
    const int QM = q_block_size > 0 ? (int)(nq / q_block_size) : 0;
    if (geometry(B, H, N, D, q_block_size, kv_block_size, q_pad_head, q_pad_tail, kv_pad_head, kv_pad_tail, QM,
                 &G) != FTA_OK)
        return 0;
    // membership bitmap KV block -> q-blocks, lse in log2 units, launch order, then
    // the split parts of dK/dV and of dQ (one region: dQ runs after dK/dV is done);
    // the dK/dV parts are sized for one K/V head per query head
    return bwd_bytes(B, H, N, G) + std::max(dq_split_bytes(B, H, G, dq_nsplit(B, H, G)),
                                            dkv_split_bytes(B, H, G, dkv_nsplit(B, H, kv_block_size, G)));
}

}  // extern "C"

namespace {
// Arguments shared by the dQ and dK/dV launches (geometry checked here).
int bwd_common(AttnArgs& a, Geo& G, const void* q, const int64_t* q_strides, const void* k,
               const int64_t* k_strides, const void* v, const int64_t* v_strides, const void* dout,
               const int64_t* do_strides, int B, int H, int Hk, int N, int D, const int32_t* merged_indices, int QM,
               int W, int q_block_size, int kv_block_size, int q_pad_head, int q_pad_tail, int kv_pad_head,
               int kv_pad_tail, float scale, const float* lse, const float* delta) {
    if (Hk <= 0 || H % Hk != 0)
        return fta::arg_error("sparse_attn_bwd: num_heads must be a multiple of num_kv_heads");
    int rc = geometry(B, H, N, D, q_block_size, kv_block_size, q_pad_head, q_pad_tail, kv_pad_head, kv_pad_tail, QM,
                      &G);
    if (rc != FTA_OK) return rc;
    if (W <= 0) return fta::arg_error("sparse_attn_bwd: qblock_topk must be positive");
    if (G.Mkv > 0x3fffffff / 32) return fta::unsupported("sparse_attn_bwd: too many KV blocks");
    a = AttnArgs{};
    a.q = (const uint16_t*)q;
    a.q_sb = q_strides[0];
    a.q_sh = q_strides[1];
    a.q_sn = q_strides[2];
    a.k = (const uint16_t*)k;
    a.k_sb = k_strides[0];
    a.k_sh = k_strides[1];
    a.k_sn = k_strides[2];
    a.v = (const uint16_t*)v;
    a.v_sb = v_strides[0];
    a.v_sh = v_strides[1];
    a.v_sn = v_strides[2];
    a.dout = (const uint16_t*)dout;
    a.d_sb = do_strides[0];
    a.d_sh = do_strides[1];
    a.d_sn = do_strides[2];
    a.merged = merged_indices;
    a.W = W;
    a.lse_in = lse;
    a.delta_in = delta;
    fill_common(a, H, N, D, q_block_size, kv_block_size, q_pad_head, kv_pad_head, scale, G);
    a.Hk = Hk;
    a.G = H / Hk;
    return FTA_OK;
}

// 64-key blocks at D 64 / 128 / 256 (the split dK/dV kernel) run in the launch
// order of fta_kv_order_kernel and the head placement of fta_head_balance_kernel
bool uses_kv_order(int kv_block_size, const Geo& G) {
    return kv_block_size > 32 && kv_block_size <= 64 && (G.Dk == 64 || G.Dk == 128 || G.Dk == 256) &&
           G.Mkv <= 4096;
}

// the head placement fta_sparse_attn_bwd_dkv left in the workspace (null if it made none)
const int32_t* dkv_head_perm(const void* workspace, int B, int H, int N, int D, int QM, int q_block_size,
                             int kv_block_size, int q_pad_head, int q_pad_tail, int kv_pad_head, int kv_pad_tail) {
    Geo G;
    if (geometry(B, H, N, D, q_block_size, kv_block_size, q_pad_head, q_pad_tail, kv_pad_head, kv_pad_tail, QM, &G) !=
            FTA_OK ||
        !uses_kv_order(kv_block_size, G))
        return nullptr;
    const char* p = (const char*)workspace + sel_bytes(B, H, G) + fta::align_up((size_t)B * H * N * sizeof(float)) +
                    fta::align_up((size_t)B * H * G.Mkv * sizeof(int32_t));
    return (const int32_t*)p + B * H;  // head work [B*Hk], then the placement
}

// dQ with an optional head placement (null: natural order)
// split_ws / split_bytes: room for dQ's split parts (null: no split)
int bwd_dq_impl(const int32_t* head_perm, const void* q, const int64_t* q_strides, const void* k, const int64_t* k_strides,
                const void* v, const int64_t* v_strides, const void* dout, const int64_t* do_strides,
                int dtype, int B, int H, int Hk, int N, int D, const int32_t* merged_indices, int QM, int W,
                int q_block_size, int kv_block_size, int q_pad_head, int q_pad_tail, int kv_pad_head,
                int kv_pad_tail, float scale, const float* lse, const float* delta, void* dq,
                const int64_t* dq_strides, void* split_ws, size_t split_avail, void* stream) {
    FTA_TRY_BEGIN
    AttnArgs a;
    Geo G;
    int rc = bwd_common(a, G, q, q_strides, k, k_strides, v, v_strides, dout, do_strides, B, H, Hk, N, D,
                        merged_indices, QM, W, q_block_size, kv_block_size, q_pad_head, q_pad_tail, kv_pad_head,
                        kv_pad_tail, scale, lse, delta);
    if (rc != FTA_OK) return rc;
    hipStream_t st = (hipStream_t)stream;
    a.head_perm = head_perm;
    a.out0 = (uint16_t*)dq;
    a.o0_sb = dq_strides[0];
    a.o0_sh = dq_strides[1];
    a.o0_sn = dq_strides[2];
    const int Tq = (G.Dk <= 128) ? 8 : 4;  // query tiles per dQ workgroup
    a.wg_per_bh = (G.Npq + 32 * Tq - 1) / (32 * Tq);
    // small grids: each workgroup's union walk in 2-4 parts, summed by fta_dq_combine_kernel
    const int ns = dq_nsplit(B, H, G);
    const bool pipe_ok = a.k_sn <= (1 << 24) && a.v_sn <= (1 << 24);
    const bool split = ns > 1 && (G.Dk > 128 || pipe_ok) && split_ws != nullptr &&
                       split_avail >= dq_split_bytes(B, H, G, ns);
    a.nsplit = split ? ns : 1;
    a.nbh = B * H;
    a.npq = G.Npq;
    a.part_o = split ? (float*)split_ws : nullptr;
    a.total = a.wg_per_bh * B * H * a.nsplit;
    if (dtype == FTA_DTYPE_BF16) return launch_dq_dt<FTA_DTYPE_BF16>(a, G.Dk, a.total, st);
    if (dtype == FTA_DTYPE_F16) return launch_dq_dt<FTA_DTYPE_F16>(a, G.Dk, a.total, st);
    return fta::arg_error("sparse_attn_bwd: dtype must be bf16 or fp16");
    FTA_TRY_END
}
}  // namespace

extern "C" {

int fta_sparse_attn_bwd_dq(const void* q, const int64_t* q_strides, const void* k, const int64_t* k_strides,
                           const void* v, const int64_t* v_strides, const void* dout, const int64_t* do_strides,
                           int dtype, int B, int H, int Hk, int N, int D, const int32_t* merged_indices, int QM, int W,
                           int q_block_size, int kv_block_size, int q_pad_head, int q_pad_tail, int kv_pad_head,
                           int kv_pad_tail, float scale, const float* lse, const float* delta, void* dq,
                           const int64_t* dq_strides, void* stream) {
    return bwd_dq_impl(nullptr, q, q_strides, k, k_strides, v, v_strides, dout, do_strides, dtype, B, H, Hk, N, D,
                       merged_indices, QM, W, q_block_size, kv_block_size, q_pad_head, q_pad_tail, kv_pad_head,
                       kv_pad_tail, scale, lse, delta, dq, dq_strides, nullptr, 0, stream);
}

int fta_sparse_attn_bwd_dkv(const void* q, const int64_t* q_strides, const void* k, const int64_t* k_strides,
                            const void* v, const int64_t* v_strides, const void* dout, const int64_t* do_strides,
                            int dtype, int B, int H, int Hk, int N, int D, const int32_t* merged_indices, int QM,
                            int W, int q_block_size, int kv_block_size, int q_pad_head, int q_pad_tail,
                            int kv_pad_head, int kv_pad_tail, float scale, const float* lse, const float* delta,
                            void* dk, const int64_t* dk_strides, void* dv, const int64_t* dv_strides, void* workspace,
                            size_t workspace_bytes, void* stream) {
    FTA_TRY_BEGIN
    AttnArgs a;
    Geo G;
    int rc = bwd_common(a, G, q, q_strides, k, k_strides, v, v_strides, dout, do_strides, B, H, Hk, N, D,
                        merged_indices, QM, W, q_block_size, kv_block_size, q_pad_head, q_pad_tail, kv_pad_head,
                        kv_pad_tail, scale, lse, delta);
    if (rc != FTA_OK) return rc;
    if (dtype != FTA_DTYPE_BF16 && dtype != FTA_DTYPE_F16)
        return fta::arg_error("sparse_attn_bwd: dtype must be bf16 or fp16");
    if (workspace_bytes < bwd_bytes(B, H, N, G)) return fta::arg_error("sparse_attn_bwd: workspace too small");
    hipStream_t st = (hipStream_t)stream;
    // membership bitmap (KV block -> q-blocks) and lse in log2 units, in the workspace
    uint32_t* sel = (uint32_t*)workspace;
    if ((rc = fta::launch_sel_bitmap(merged_indices, B * H, QM, W, G.Mkv, sel, st)) != FTA_OK) return rc;
    float* lse2 = (float*)((char*)workspace + sel_bytes(B, H, G));
    const int64_t nl = (int64_t)B * H * N;
    hipLaunchKernelGGL(fta_lse2_kernel, dim3((unsigned)((nl + 255) / 256)), dim3(256), 0, st, lse, lse2, nl);
    if ((rc = fta::check_launch("fta_lse2_kernel")) != FTA_OK) return rc;
    a.sel = sel;
    a.lse2_in = lse2;
    // 64-key blocks at D 64 / 128 (the split kernel): launch in first-q-block order
    if (uses_kv_order(kv_block_size, G)) {
        int32_t* order = (int32_t*)((char*)lse2 + fta::align_up((size_t)B * H * N * sizeof(float)));
        int32_t* head_work = (int32_t*)((char*)order + fta::align_up((size_t)B * H * G.Mkv * sizeof(int32_t)));
        int32_t* head_perm = head_work + B * Hk;
        if ((rc = fta::launch_kv_order(sel, B, H, Hk, G.Mkv, (QM + 31) / 32, order, head_work, head_perm, st)) !=
            FTA_OK)
            return rc;
        a.kv_order = order;
        a.head_perm = head_perm;
    }
    a.out0 = (uint16_t*)dk;
    a.o0_sb = dk_strides[0];
    a.o0_sh = dk_strides[1];
    a.o0_sn = dk_strides[2];
    a.out1 = (uint16_t*)dv;
    a.o1_sb = dv_strides[0];
    a.o1_sh = dv_strides[1];
    a.o1_sn = dv_strides[2];
    const int Tb = (kv_block_size + 31) / 32;
    const int ntiles = G.Mkv * Tb;
    // small grids: each KV block's chunk list in parts (split kernel), summed by
    // fta_dkv_combine_kernel, when the workspace has room for the parts
    const int ns = dkv_nsplit(B, Hk, kv_block_size, G);
    const size_t used = bwd_bytes(B, H, N, G);
    const bool split = ns > 1 && workspace_bytes >= used + dkv_split_bytes(B, Hk, G, ns);
    a.nsplit = split ? ns : 1;
    a.nbh = B * Hk;
    a.npq = G.Mkv * 64;
    a.part_o = split ? (float*)((char*)workspace + used) : nullptr;
    // one dK/dV WG set per K/V head; each walks the G query heads that share it
    if (dtype == FTA_DTYPE_BF16) return launch_dkv_dt<FTA_DTYPE_BF16>(a, G.Dk, Tb, B, Hk, ntiles, st);
    return launch_dkv_dt<FTA_DTYPE_F16>(a, G.Dk, Tb, B, Hk, ntiles, st);
    FTA_TRY_END
}

int fta_sparse_attn_bwd_gqa(const void* q, const int64_t* q_strides, const void* k, const int64_t* k_strides,
                            const void* v, const int64_t* v_strides, const void* dout, const int64_t* do_strides,
                            int dtype, int B, int H, int Hk, int N, int D, const int32_t* merged_indices, int QM,
                            int W, int q_block_size, int kv_block_size, int q_pad_head, int q_pad_tail,
                            int kv_pad_head, int kv_pad_tail, float scale, const float* lse, const float* delta,
                            void* dq, const int64_t* dq_strides, void* dk, const int64_t* dk_strides, void* dv,
                            const int64_t* dv_strides, void* workspace, size_t workspace_bytes, void* stream) {
    // dK / dV first: its launch-order pass also places the heads on XCDs by their
    // work, which dQ reuses when every query head has its own K / V head
    int rc = fta_sparse_attn_bwd_dkv(q, q_strides, k, k_strides, v, v_strides, dout, do_strides, dtype, B, H, Hk, N,
                                     D, merged_indices, QM, W, q_block_size, kv_block_size, q_pad_head, q_pad_tail,
                                     kv_pad_head, kv_pad_tail, scale, lse, delta, dk, dk_strides, dv, dv_strides,
                                     workspace, workspace_bytes, stream);
    if (rc != FTA_OK) return rc;
    const int32_t* perm = (Hk == H) ? dkv_head_perm(workspace, B, H, N, D, QM, q_block_size, kv_block_size,
                                                    q_pad_head, q_pad_tail, kv_pad_head, kv_pad_tail)
                                    : nullptr;
    // dQ's split parts go after the dK/dV pass's bytes (it has validated the geometry)
    Geo G;
    geometry(B, H, N, D, q_block_size, kv_block_size, q_pad_head, q_pad_tail, kv_pad_head, kv_pad_tail, QM, &G);
    const size_t used = bwd_bytes(B, H, N, G);
    void* split_ws = workspace_bytes > used ? (char*)workspace + used : nullptr;
    return bwd_dq_impl(perm, q, q_strides, k, k_strides, v, v_strides, dout, do_strides, dtype, B, H, Hk, N, D,
                       merged_indices, QM, W, q_block_size, kv_block_size, q_pad_head, q_pad_tail, kv_pad_head,
                       kv_pad_tail, scale, lse, delta, dq, dq_strides, split_ws,
                       split_ws ? workspace_bytes - used : 0, stream);
}

int fta_sparse_attn_fwd(const void* q, const int64_t* q_strides, const void* k, const int64_t* k_strides,
                        const void* v, const int64_t* v_strides, int dtype, int B, int H, int N, int D,
                        const int32_t* merged_indices, int QM, int W, int q_block_size, int kv_block_size,
                        int q_pad_head, int q_pad_tail, int kv_pad_head, int kv_pad_tail, float scale, void* o,
                        const int64_t* o_strides, float* lse, void* workspace, size_t workspace_bytes,
                        void* stream) {
    return fta_sparse_attn_fwd_gqa(q, q_strides, k, k_strides, v, v_strides, dtype, B, H, H, N, D, merged_indices,
                                   QM, W, q_block_size, kv_block_size, q_pad_head, q_pad_tail, kv_pad_head,
                                   kv_pad_tail, scale, o, o_strides, lse, workspace, workspace_bytes, stream);
}

int fta_sparse_attn_bwd(const void* q, const int64_t* q_strides, const void* k, const int64_t* k_strides,
                        const void* v, const int64_t* v_strides, const void* dout, const int64_t* do_strides,
                        int dtype, int B, int H, int N, int D, const int32_t* merged_indices, int QM, int W,
                        int q_block_size, int kv_block_size, int q_pad_head, int q_pad_tail, int kv_pad_head,
                        int kv_pad_tail, float scale, const float* lse, const float* delta, void* dq,
                        const int64_t* dq_strides, void* dk, const int64_t* dk_strides, void* dv,
                        const int64_t* dv_strides, void* workspace, size_t workspace_bytes, void* stream) {
    return fta_sparse_attn_bwd_gqa(q, q_strides, k, k_strides, v, v_strides, dout, do_strides, dtype, B, H, H, N, D,
                                   merged_indices, QM, W, q_block_size, kv_block_size, q_pad_head, q_pad_tail,
                                   kv_pad_head, kv_pad_tail, scale, lse, delta, dq, dq_strides, dk, dk_strides, dv,
                                   dv_strides, workspace, workspace_bytes, stream);
}

}  // extern "C"

// ----------------------------------------------------------------------------
// Allocation-free backward.  Its workspace is this file-scope device array
// (each GPU that loads the library holds its own copy until the process ends).
// Host code never passes `scratch` itself to a kernel or a copy: the name is a
// host-side stand-in; the array's device address comes from
// hipGetSymbolAddress, taken once per device on the first call there.
// ----------------------------------------------------------------------------
static __device__ __align__(256) unsigned char scratch[FTA_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

int scratch_address(void** out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) {
        fta::set_error(std::string("sparse_attn_bwd_noalloc: hipGetDevice: ") + hipGetErrorString(e));
        return FTA_ERR_HIP;
    }
    if (dev < 0 || dev >= kMaxDevices) return fta::unsupported("sparse_attn_bwd_noalloc: device index >= 64");
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_ptr[dev] == nullptr) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || p == nullptr) {
            fta::set_error(std::string("sparse_attn_bwd_noalloc: hipGetSymbolAddress(scratch): ") +
                           hipGetErrorString(e));
            return FTA_ERR_HIP;
        }
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return FTA_OK;
}
}  // namespace

extern "C" int fta_sparse_attn_bwd_noalloc(
    const void* q, const int64_t* q_strides, const void* k, const int64_t* k_strides, const void* v,
    const int64_t* v_strides, const void* dout, const int64_t* do_strides, int dtype, int B, int H, int Hk, int N,
    int D, const int32_t* merged_indices, int QM, int W, int q_block_size, int kv_block_size, int q_pad_head,
    int q_pad_tail, int kv_pad_head, int kv_pad_tail, float scale, const float* lse, const float* delta, void* dq,
    const int64_t* dq_strides, void* dk, const int64_t* dk_strides, void* dv, const int64_t* dv_strides,
    void* stream) {
    FTA_TRY_BEGIN
    // the bitmap, log2 lse and launch order must fit; dQ's split parts are used
    // only when they fit as well (fta_sparse_attn_bwd_gqa checks the room left)
    Geo G;
    size_t need = fta_sparse_attn_bwd_workspace_size(B, H, N, D, q_block_size, kv_block_size, q_pad_head,
                                                     q_pad_tail, kv_pad_head, kv_pad_tail);
    const int64_t nq = (int64_t)q_pad_head + N + q_pad_tail;
    if (q_block_size > 0 && geometry(B, H, N, D, q_block_size, kv_block_size, q_pad_head, q_pad_tail, kv_pad_head,
                                     kv_pad_tail, (int)(nq / q_block_size), &G) == FTA_OK)
        need = bwd_bytes(B, H, N, G);
    if (need > (size_t)FTA_NOALLOC_SCRATCH_BYTES)
        return fta::unsupported(
            "sparse_attn_bwd_noalloc: the problem needs more scratch than FTA_NOALLOC_SCRATCH_BYTES "
            "(membership bitmap + log2 lse); use fta_sparse_attn_bwd_gqa with a caller workspace");
    void* ws = nullptr;
    const int rc = scratch_address(&ws);
    if (rc != FTA_OK) return rc;
    // every scratch byte the kernels read is written earlier in the same call
    // (the bitmap is built whole, the log2 lse is converted in full), so no
    // clearing is needed; calls that overlap on one GPU race on the array
    return fta_sparse_attn_bwd_gqa(q, q_strides, k, k_strides, v, v_strides, dout, do_strides, dtype, B, H, Hk, N,
                                   D, merged_indices, QM, W, q_block_size, kv_block_size, q_pad_head, q_pad_tail,
                                   kv_pad_head, kv_pad_tail, scale, lse, delta, dq, dq_strides, dk, dk_strides, dv,
                                   dv_strides, ws, (size_t)FTA_NOALLOC_SCRATCH_BYTES, stream);
    FTA_TRY_END
}
