// Block scoring and top-k selection for gfx950.
//
// Block scoring (reference: flash_topk_attn_v2/csrc/block_score_kernel.cu:19-314,
// flash_topk_attn_v2/block_score.py:295-366) computes, for every query t and
// virtual score block j of b keys,
//     score[t, j] = sum_{keys i in block j} softmax(q_t K^T / sqrt(D))_i .
// Here it is done in two stages:
//   1. fta_block_score_lse_kernel streams K once per 256-query tile and emits the
//      per-block log2-sum-exp  lse2[j, t] = log2 sum_{i in j} 2^{c s_i}
//      (c = scale * log2 e) plus the row total lse2[t]; both fp32.  Layout of
//      the per-block values is [BH][M][N] so that lanes (= queries) store
//      contiguously.
//   2. score = 2^{lse2[j, t] - lse2[t]}, either materialised by
//      fta_block_normalize_kernel ([BH][N][M], the public block-score tensor) or
//      consumed directly by the top-k selector (fused path, no [BH][N][M] array).
//
// Top-k selection (reference: flash_topk_attn_v2/topk_select.py:128-182 and
// csrc/topk_select_kernel.cu:7-131) ranks blocks by avg = raw / valid_count,
// ties to the lower block index, keeps the first max_topk, and truncates after
// the first position whose sequential fp32 cumulative sum of avg * valid_count
// reaches the threshold.
#include "fta_common.h"


// ----------------------------------------------------------------------------
// Stage 1: per-block log2-sum-exp.
// WG = 4 waves, each wave owns 64 queries (two 32-column MFMA tiles); the WG
// stages 64-key chunks of K in LDS (double-buffered).  S^T = K Q^T so that each
// lane holds 16 keys of one query per 32x32 tile and the reduction over keys is
// in-lane plus one exchange with lane ^ 32.
// ----------------------------------------------------------------------------
template <int DT, int D>
__global__ __launch_bounds__(256, (D > 160) ? 1 : 2) void fta_block_score_lse_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
    int64_t q_sb, int64_t q_sh, int64_t q_sn, int64_t k_sb, int64_t k_sh, int64_t k_sn,
    int H, int N, int Dreal, int M, int bsz, int pad_head, int pad_tail, float c,
    float* __restrict__ blk_lse, float* __restrict__ row_lse, int qtiles, int total, int kgroups,
    int32_t* __restrict__ tau_idx) {
    using E = Elem<DT>;
    constexpr int KS = D / 16;
    constexpr int ROW = D + 8;  // +16 B per LDS row against bank conflicts
    constexpr int SEGS = D / 8;
    constexpr int LOADS = (64 * SEGS) / 256;
    static_assert((64 * SEGS) % 256 == 0, "D must be a multiple of 32");
    __shared__ __align__(16) uint16_t sk[2][64 * ROW];

    const int wg = fta_xcd_remap(blockIdx.x, total);
    const int bh = wg / qtiles;
    const int qt = wg - bh * qtiles;
    const int b = bh / H, h = bh - (bh / H) * H;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int qbase = qt * 256 + wave * 64;
    const uint16_t* qp = q + b * q_sb + h * q_sh;
    const uint16_t* kp = k + b * k_sb + h * k_sh;

    uint4 qf[2][KS];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        const int qi = qbase + t * 32 + (lane & 31);
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            const int d = ks * 16 + (lane >> 5) * 8;
            qf[t][ks] = (qi < N && d < Dreal) ? *reinterpret_cast<const uint4*>(qp + (int64_t)qi * q_sn + d)
                                              : fta_zero4();
        }
    }

    const int nchunk = (bsz + 63) >> 6;
    const int total_it = M * nchunk;
    uint4 stage[LOADS];

    auto load_chunk = [&](int it) {
        const int m = it / nchunk, ch = it - (it / nchunk) * nchunk;
        const int kb = m * bsz - pad_head + ch * 64;
        const int rem = bsz - ch * 64;
#pragma unroll
        for (int i = 0; i < LOADS; ++i) {
            const int s = tid + i * 256;
            const int row = s / SEGS, seg = s - (s / SEGS) * SEGS;
            const int t = kb + row;
            const bool ok = row < rem && t >= 0 && t < N && seg * 8 < Dreal;
            stage[i] = ok ? *reinterpret_cast<const uint4*>(kp + (int64_t)t * k_sn + seg * 8) : fta_zero4();
        }
    };
    auto store_chunk = [&](int buf) {
#pragma unroll
        for (int i = 0; i < LOADS; ++i) {
            const int s = tid + i * 256;
            const int row = s / SEGS, seg = s - (s / SEGS) * SEGS;
            *reinterpret_cast<uint4*>(&sk[buf][row * ROW + seg * 8]) = stage[i];
        }
    };

    float m_run[2] = {-FTA_INF, -FTA_INF}, L_run[2] = {0.f, 0.f};
    float mb[2] = {-FTA_INF, -FTA_INF}, lb[2] = {0.f, 0.f};
    // Lower bound for the top-k selector: split the M blocks into kgroups
    // groups, keep each group's best block (by log2 average mass) and the worst
    // of those group maxima -- at least kgroups blocks are at least that good.
    float gkey = -FTA_INF, tkey = FTA_INF;
    int gidx = 0, tidx = 0, curg = -1;
    const float adj_head = (pad_head > 0) ? fta_log2((float)bsz / (float)(bsz - pad_head)) : 0.f;
    const float adj_tail = (pad_tail > 0) ? fta_log2((float)bsz / (float)(bsz - pad_tail)) : 0.f;

    load_chunk(0);
    store_chunk(0);
    __syncthreads();

    for (int it = 0; it < total_it; ++it) {
        const int buf = it & 1;
        if (it + 1 < total_it) load_chunk(it + 1);
        const int m = it / nchunk, ch = it - (it / nchunk) * nchunk;
        const int kb = m * bsz - pad_head + ch * 64;
        const int rem = bsz - ch * 64;
        const bool two = rem > 32;

        f32x16 acc[2][2];
#pragma unroll
        for (int s = 0; s < 2; ++s)
#pragma unroll
            for (int t = 0; t < 2; ++t)
#pragma unroll
                for (int i = 0; i < 16; ++i) acc[s][t][i] = 0.f;

        const uint16_t* base = &sk[buf][0];
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            const uint4 a0 =
                *reinterpret_cast<const uint4*>(base + (lane & 31) * ROW + ks * 16 + (lane >> 5) * 8);
            acc[0][0] = E::mma(a0, qf[0][ks], acc[0][0]);
            acc[0][1] = E::mma(a0, qf[1][ks], acc[0][1]);
        }
        if (two) {
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                const uint4 a1 = *reinterpret_cast<const uint4*>(base + (32 + (lane & 31)) * ROW + ks * 16 +
                                                                 (lane >> 5) * 8);
                acc[1][0] = E::mma(a1, qf[0][ks], acc[1][0]);
                acc[1][1] = E::mma(a1, qf[1][ks], acc[1][1]);
            }
        }

        const bool need_mask = kb < 0 || kb + 64 > N || rem < 64;
        if (need_mask) {
#pragma unroll
            for (int s = 0; s < 2; ++s)
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const int rel = s * 32 + c_row(i, lane);
                    const int t = kb + rel;
                    if (rel >= rem || t < 0 || t >= N) {
                        acc[s][0][i] = -FTA_INF;
                        acc[s][1][i] = -FTA_INF;
                    }
                }
        }

#pragma unroll
        for (int t = 0; t < 2; ++t) {
            float mx = acc[0][t][0];
#pragma unroll
            for (int i = 1; i < 16; ++i) mx = fmaxf(mx, acc[0][t][i]);
            if (two) {
#pragma unroll
                for (int i = 0; i < 16; ++i) mx = fmaxf(mx, acc[1][t][i]);
            }
            mx = fmaxf(mx, fta_xor32(mx));
            const float mref = (ch == 0) ? mx : fmaxf(mb[t], mx);
            const float mr = (mref == -FTA_INF) ? 0.f : mref;
            const float mc = mr * c;
            float sum = 0.f;
#pragma unroll
            for (int i = 0; i < 16; ++i) sum += fta_exp2(fmaf(acc[0][t][i], c, -mc));
            if (two) {
#pragma unroll
                for (int i = 0; i < 16; ++i) sum += fta_exp2(fmaf(acc[1][t][i], c, -mc));
            }
            sum += fta_xor32(sum);
            lb[t] = (ch == 0) ? sum : fmaf(lb[t], fta_exp2((mb[t] - mr) * c), sum);
            mb[t] = mref;
        }

        if (ch == nchunk - 1) {
            float lse_b[2];
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                lse_b[t] = (lb[t] > 0.f) ? fmaf(mb[t], c, fta_log2(lb[t])) : -FTA_INF;
                if (lb[t] > 0.f) {
                    const float mn = fmaxf(m_run[t], mb[t]);
                    L_run[t] = L_run[t] * fta_exp2((m_run[t] - mn) * c) + lb[t] * fta_exp2((mb[t] - mn) * c);
                    m_run[t] = mn;
                }
            }
            const int qi = qbase + lane;
            const float mine = (lane < 32) ? lse_b[0] : lse_b[1];
            if (qi < N) blk_lse[((int64_t)bh * M + m) * N + qi] = mine;
            if (kgroups > 0) {
                const int gm = (int)(((int64_t)m * kgroups) / M);
                float key = mine;
                if (m == 0) key += adj_head;
                if (m == M - 1) key += adj_tail;
                if (gm != curg) {
                    if (curg >= 0 && gkey < tkey) {
                        tkey = gkey;
                        tidx = gidx;
                    }
                    curg = gm;
                    gkey = key;
                    gidx = m;
                } else if (key > gkey) {
                    gkey = key;
                    gidx = m;
                }
            }
        }

        if (it + 1 < total_it) store_chunk(buf ^ 1);
        __syncthreads();
    }

    const int qi = qbase + lane;
    if (qi < N) {
        const int t = lane >> 5;
        const float mr = (t == 0) ? m_run[0] : m_run[1];
        const float Lr = (t == 0) ? L_run[0] : L_run[1];
        row_lse[(int64_t)bh * N + qi] = (Lr > 0.f) ? fmaf(mr, c, fta_log2(Lr)) : -FTA_INF;
        if (kgroups > 0) {
            if (curg >= 0 && gkey < tkey) tidx = gidx;
            tau_idx[(int64_t)bh * N + qi] = tidx;
        }
    }
}


// Sum of 2^{c v_i - r} over n values: all exps are issued before any add and the
// adds form a tree, so no add waits on the exp issued just before it.
template <int NV>
__device__ __forceinline__ float fta_sum_exp2(const float* v, float c, float r) {
    float e[NV];
#pragma unroll
    for (int i = 0; i < NV; ++i) e[i] = fta_exp2(fmaf(v[i], c, -r));
#pragma unroll
    for (int w = 1; w < NV; w <<= 1)
#pragma unroll
        for (int i = 0; i + w < NV; i += 2 * w) e[i] += e[i + w];
    return e[0];
}
// ----------------------------------------------------------------------------
// Stage 1, blocks of at most 64 keys (one LDS chunk per block).  Same tiling
// as above, but the per-block max pass is replaced by a running per-row log2
// reference R: p = 2^{c s - R}, block total = exchange of two lane halves.
// R starts at -inf, which makes the first block take the exact path (per-block
// max, as above); it is re-based onto a block's log-sum whenever a block
// total exceeds 2^40, and any non-finite or > 2^100 total (a logit more than
// ~100/c above the reference) recomputes that block exactly.  Blocks far below
// R lose mass to underflow only when they sit more than 2^-126 below R, i.e.
// when their score is below fp32 resolution anyway.
// ----------------------------------------------------------------------------
template <int DT, int D, int QT>
__global__ __launch_bounds__(256 * (2 / QT), (D > 160) ? 1 : 2) void fta_block_score_lse_fast_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
    int64_t q_sb, int64_t q_sh, int64_t q_sn, int64_t k_sb, int64_t k_sh, int64_t k_sn,
    int H, int N, int Dreal, int M, int bsz, int pad_head, int pad_tail, float c,
    float* __restrict__ blk_lse, float* __restrict__ row_lse, int qtiles, int total, int kgroups,
    int32_t* __restrict__ tau_idx) {
    using E = Elem<DT>;
    constexpr int KS = D / 16;
    constexpr int ROW = D + 8;
    constexpr int SEGS = D / 8;
    constexpr int NTHR = 256 * (2 / QT);
    constexpr int LOADS = (64 * SEGS + NTHR - 1) / NTHR;
    static_assert(QT == 1 || QT == 2, "one or two query tiles per wave");
    __shared__ __align__(16) uint16_t sk[2][64 * ROW];

    const int wg = fta_xcd_remap(blockIdx.x, total);
    const int bh = wg / qtiles;
    const int qt = wg - bh * qtiles;
    const int b = bh / H, h = bh - (bh / H) * H;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int qbase = qt * 256 + wave * 32 * QT;
    const uint16_t* qp = q + b * q_sb + h * q_sh;
    const uint16_t* kp = k + b * k_sb + h * k_sh;

    uint4 qf[QT][KS];
#pragma unroll
    for (int t = 0; t < QT; ++t) {
        const int qi = qbase + t * 32 + (lane & 31);
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            const int d = ks * 16 + (lane >> 5) * 8;
            qf[t][ks] = (qi < N && d < Dreal) ? *reinterpret_cast<const uint4*>(qp + (int64_t)qi * q_sn + d)
                                              : fta_zero4();
        }
    }

    uint4 stage[LOADS];
    auto load_block = [&](int m) {
        const int kb = m * bsz - pad_head;
        if (kb >= 0 && kb + 64 <= N && bsz == 64 && Dreal == D) {
            // interior block: no bounds checks
#pragma unroll
            for (int i = 0; i < LOADS; ++i) {
                const int s = tid + i * NTHR;
                const int row = s / SEGS, seg = s - (s / SEGS) * SEGS;
                if (s < 64 * SEGS) stage[i] = *reinterpret_cast<const uint4*>(kp + (int64_t)(kb + row) * k_sn + seg * 8);
            }
        } else {
#pragma unroll
            for (int i = 0; i < LOADS; ++i) {
                const int s = tid + i * NTHR;
                const int row = s / SEGS, seg = s - (s / SEGS) * SEGS;
                const int t = kb + row;
                const bool ok = s < 64 * SEGS && row < bsz && t >= 0 && t < N && seg * 8 < Dreal;
                const int tc = min(max(t, 0), N - 1);
                const uint4 v = *reinterpret_cast<const uint4*>(kp + (int64_t)tc * k_sn + (ok ? seg * 8 : 0));
                stage[i] = ok ? v : fta_zero4();
            }
        }
    };
    auto store_block = [&](int buf) {
#pragma unroll
        for (int i = 0; i < LOADS; ++i) {
            const int s = tid + i * NTHR;
            const int row = s / SEGS, seg = s - (s / SEGS) * SEGS;
            if (s < 64 * SEGS) *reinterpret_cast<uint4*>(&sk[buf][row * ROW + seg * 8]) = stage[i];
        }
    };

    float R[2] = {-FTA_INF, -FTA_INF}, L[2] = {0.f, 0.f};
    float gkey = -FTA_INF, tkey = FTA_INF;
    int gidx = 0, tidx = 0, curg = -1, next_start = 0;
    const float adj_head = (pad_head > 0) ? fta_log2((float)bsz / (float)(bsz - pad_head)) : 0.f;
    const float adj_tail = (pad_tail > 0) ? fta_log2((float)bsz / (float)(bsz - pad_tail)) : 0.f;
    const bool two = bsz > 32;
    const int kr0 = (lane & 31) * ROW + (lane >> 5) * 8;

    load_block(0);
    store_block(0);
    __syncthreads();

    for (int m = 0; m < M; ++m) {
        const int buf = m & 1;
        if (m + 1 < M) load_block(m + 1);
        const int kb = m * bsz - pad_head;

        f32x16 acc[2][2];
        const f32x16 zacc = {};
        const uint16_t* base = &sk[buf][0];
        __builtin_amdgcn_s_setprio(1);  // keep the matrix core fed while the co-resident wave runs VALU
        if (two) {
            uint4 a0 = *reinterpret_cast<const uint4*>(base + kr0);
            uint4 a1 = *reinterpret_cast<const uint4*>(base + kr0 + 32 * ROW);
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                uint4 n0 = a0, n1 = a1;
                if (ks + 1 < KS) {
                    n0 = *reinterpret_cast<const uint4*>(base + kr0 + (ks + 1) * 16);
                    n1 = *reinterpret_cast<const uint4*>(base + kr0 + 32 * ROW + (ks + 1) * 16);
                }
                acc[0][0] = E::mma(a0, qf[0][ks], ks ? acc[0][0] : zacc);
                if (QT == 2) acc[0][1] = E::mma(a0, qf[QT - 1][ks], ks ? acc[0][1] : zacc);
                acc[1][0] = E::mma(a1, qf[0][ks], ks ? acc[1][0] : zacc);
                if (QT == 2) acc[1][1] = E::mma(a1, qf[QT - 1][ks], ks ? acc[1][1] : zacc);
                a0 = n0;
                a1 = n1;
            }
        } else {
            uint4 a0 = *reinterpret_cast<const uint4*>(base + kr0);
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                uint4 n0 = a0;
                if (ks + 1 < KS) n0 = *reinterpret_cast<const uint4*>(base + kr0 + (ks + 1) * 16);
                acc[0][0] = E::mma(a0, qf[0][ks], ks ? acc[0][0] : zacc);
                if (QT == 2) acc[0][1] = E::mma(a0, qf[QT - 1][ks], ks ? acc[0][1] : zacc);
                a0 = n0;
            }
            acc[1][0] = zacc;
            acc[1][1] = zacc;
        }

        __builtin_amdgcn_s_setprio(0);
        if (kb < 0 || kb + 64 > N || bsz < 64) {
#pragma unroll
            for (int s = 0; s < 2; ++s)
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const int rel = s * 32 + c_row(i, lane);
                    const int t = kb + rel;
                    if (rel >= bsz || t < 0 || t >= N) {
                        acc[s][0][i] = -FTA_INF;
                        acc[s][1][i] = -FTA_INF;
                    }
                }
        }

        float tot[2];
#pragma unroll
        for (int t = 0; t < QT; ++t) {
            float v[32];
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                v[i] = acc[0][t][i];
                v[16 + i] = acc[1][t][i];
            }
            const float part = two ? fta_sum_exp2<32>(v, c, R[t]) : fta_sum_exp2<16>(v, c, R[t]);
            tot[t] = part + fta_xor32(part);
        }
        const bool bad = !(tot[0] < 0x1p100f) || (QT == 2 && !(tot[QT - 1] < 0x1p100f));
        if (__ballot(bad) != 0ull) {
            // exact path: reference = this block's max
#pragma unroll
            for (int t = 0; t < QT; ++t) {
                float mx = acc[0][t][0];
#pragma unroll
                for (int i = 1; i < 16; ++i) mx = fmaxf(mx, acc[0][t][i]);
                if (two) {
#pragma unroll
                    for (int i = 0; i < 16; ++i) mx = fmaxf(mx, acc[1][t][i]);
                }
                mx = fmaxf(mx, fta_xor32(mx));
                const float Rn = (mx == -FTA_INF) ? 0.f : mx * c;
                L[t] = (L[t] > 0.f) ? L[t] * fta_exp2(R[t] - Rn) : 0.f;
                R[t] = Rn;
                float v[32];
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    v[i] = acc[0][t][i];
                    v[16 + i] = acc[1][t][i];
                }
                const float part = two ? fta_sum_exp2<32>(v, c, Rn) : fta_sum_exp2<16>(v, c, Rn);
                tot[t] = part + fta_xor32(part);
            }
        }
        float lse_b[2];
#pragma unroll
        for (int t = 0; t < QT; ++t) {
            lse_b[t] = (tot[t] > 0.f) ? R[t] + fta_log2(tot[t]) : -FTA_INF;
            L[t] += tot[t];
            if (tot[t] > 0x1p40f) {
                const float Rn = lse_b[t];
                L[t] *= fta_exp2(R[t] - Rn);
                R[t] = Rn;
            }
        }
        // lane owns query (lane & 31) of tile (lane >> 5) (two tiles) or of the only tile
        const int qi = qbase + ((QT == 2) ? lane : (lane & 31));
        const float mine = (QT == 2 && lane >= 32) ? lse_b[QT - 1] : lse_b[0];
        if (qi < N && (QT == 2 || lane < 32)) blk_lse[((int64_t)bh * M + m) * N + qi] = mine;
        if (kgroups > 0) {
            float key = mine;
            if (m == 0) key += adj_head;
            if (m == M - 1) key += adj_tail;
            if (m == next_start) {
                if (curg >= 0 && gkey < tkey) {
                    tkey = gkey;
                    tidx = gidx;
                }
                ++curg;
                next_start = ((curg + 1) * M + kgroups - 1) / kgroups;  // first block of group curg + 1
                gkey = key;
                gidx = m;
            } else if (key > gkey) {
                gkey = key;
                gidx = m;
            }
        }

        if (m + 1 < M) store_block(buf ^ 1);
        __syncthreads();
    }

    const int qi = qbase + ((QT == 2) ? lane : (lane & 31));
    if (qi < N && (QT == 2 || lane < 32)) {
        const bool t1 = QT == 2 && lane >= 32;
        const float Rr = t1 ? R[QT - 1] : R[0];
        const float Lr = t1 ? L[QT - 1] : L[0];
        row_lse[(int64_t)bh * N + qi] = (Lr > 0.f) ? Rr + fta_log2(Lr) : -FTA_INF;
        if (kgroups > 0) {
            if (curg >= 0 && gkey < tkey) tidx = gidx;
            tau_idx[(int64_t)bh * N + qi] = tidx;
        }
    }
}

// ----------------------------------------------------------------------------
// Stage 1, software-pipelined variant for 64-key blocks and D in {64, 128}.
// Numerics are those of fta_block_score_lse_fast_kernel with two query tiles
// per wave (same running reference R, exact fallback, rebase, tau tracking and
// summation order: the 32-term tree per block is tree16(keys 0..31) +
// tree16(keys 32..63), computed here one half at a time).  The schedule differs:
//  * K blocks are gathered by LDS DMA into four swizzled buffers, up to three
//    blocks ahead of use, so no staging registers or LDS stores are needed;
//  * work is pipelined by half blocks (32 keys): the 16 MFMAs of the next half
//    are issued interleaved with the exp / sum work of the current half
//    (sched_group_barrier), so a wave keeps the matrix core and the VALU busy
//    together; only two half-block score sets are live, which keeps two waves
//    per SIMD;
//  * the rare exact path recomputes block m's scores from its LDS buffer.
// ----------------------------------------------------------------------------
template <int D>
struct ScorePipeShape {
    static constexpr int QSEG = D / 8;
    static constexpr int SLOTS = 64 * QSEG;  // 16-byte slots per K block
    static constexpr int LQ = SLOTS / 256;   // DMA instructions per wave per block (4 waves)
    static constexpr int NBUF = 4;
    static constexpr int BUF_B = SLOTS * 16;
    static_assert(SLOTS % 256 == 0, "whole DMA instructions per wave");
};

// Candidate streams (template NG > 0, top-k lists of at most 32 blocks):
// instead of the [BH][M][N] per-block values, each wave appends, per block, an
// entry (value, lane << 16 | m) for every query of the wave for which the block
// can still be in the top-k, compacted in lane order into the wave's chunks of
// the pool; the wave's entry count goes to count[wave].  A block is dropped for
// a query when at least m_out earlier blocks rank strictly above it: each query
// keeps, in LDS, the GT largest ranking keys (block value + log2(b / valid
// count)) of NG interleaved block groups (m mod NG; NG x GT = 4 x 2 for m_out
// <= 8, 4 x 4 for <= 16, 8 x 4 in fp16 for <= 32); the smallest kept key over
// the groups bounds NG GT >= m_out earlier blocks from below.  The bound is
// refreshed once per NG blocks and lowered by a
// margin far above fp32 exp2 / log2 rounding, and partial edge blocks always
// pass, so the final selection over the streams equals the one over all
// blocks.  tau_key[row] receives the final bound (at least m_out blocks rank
// at or above it).
constexpr int kStreamMaxTopk = 32;
// Entries per stream chunk (a multiple of the selector's 256-entry steps).
constexpr int kStreamChunk = 1024;

// Filter margin in log2 units.  A block is dropped only when its key is below
// the bound by more than this, while at least m_out blocks have keys at or above
// the bound; the selector ranks blocks by avg = 2^(fl(value - rl)) / b.  With
// |value - rl| <= ~101 log2 units (the range that matters, see the end-of-tile
// check), fl(value - rl) is off by at most 2^-24 * 128 = 2^-17 and v_exp_f32 by
// about 1 ulp (2^-23 relative), so keys 2^-14 apart give strictly ordered
// normal averages (8x slack); the relative term covers the rounding of the
// subtraction below for large keys.
__device__ __forceinline__ float fta_stream_margin(float b) { return b - (0x1p-14f + fabsf(b) * 0x1p-20f); }

// Arguments of the pipelined scoring kernel (one struct, passed by value).
struct ScoreArgs {
    const uint16_t* q;
    const uint16_t* k;
    int64_t q_sb, q_sh, q_sn, k_sb, k_sh, k_sn;
    int H, N, Dreal, M, bsz, pad_head, pad_tail;
    float c;
    // NG = 0: per-block values.  blk_ld = 0 writes the [B*H][M][N] array at
    // blk_lse; blk_ld > 0 writes the tile's own [M][blk_ld] slot at blk_lse
    // (query qt * 256 + j at column j).
    float* blk_lse;
    int blk_ld;
    float* row_lse;
    int qtiles, total, kgroups;
    int32_t* tau_idx;
    // NG > 0: candidate streams in chunks of kStreamChunk entries.  Wave w's
    // first chunk is chunk w of `pool`; further chunks are taken from the
    // counter pool_ctr (chunk ids waves + counter value, below pool_chunks) and
    // recorded in chunk_tab[w][1 ..].  count[w] = the wave's entry count, or -1
    // when the pool ran out (the wave's tile is then scored again by the
    // fallback kernel).
    uint2* pool;
    int* count;
    float* tau_key;
    int* chunk_tab;
    int* pool_ctr;
    int pool_chunks, maxch;
};

// Group state of the candidate-stream filter: per query and block group, the GT
// largest ranking keys seen, descending, as fp32 (GH = false) or as fp16 (GH =
// true: half the LDS; keys relative to the query's first block key, and the
// stored values may exceed them by the fp16 rounding, 2^-11 relative, which
// the bound's margin covers).
template <int GB>
struct GroupRaw;
template <>
struct GroupRaw<8> {
    using type = uint2;
};
template <>
struct GroupRaw<16> {
    using type = uint4;
};
__device__ __forceinline__ float fta_h2f(uint32_t bits) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(bits & 0xffffu));
}
__device__ __forceinline__ uint32_t fta_f2h2(float lo, float hi) {
    return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)lo) |
           ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)hi) << 16);
}

// SB = 64-key LDS chunks per score block: 1 (b = 64) or 2 (b = 128).  The
// pipeline runs over chunks u (keys u * 64 - pad_head ...); a block's value is
// formed at its last chunk from the chunk totals, all taken against the row's
// running reference R (an exact-path re-reference inside a block rescales the
// block's earlier chunks, as it rescales the row total).
template <int DT, int D, int NG, int GT = 2, bool GH = false, int SB = 1>
__device__ __forceinline__ void fta_score_tile(const ScoreArgs& a, const int wg) {
    const uint16_t* __restrict__ q = a.q;
    const uint16_t* __restrict__ k = a.k;
    const int64_t q_sb = a.q_sb, q_sh = a.q_sh, q_sn = a.q_sn, k_sb = a.k_sb, k_sh = a.k_sh, k_sn = a.k_sn;
    const int H = a.H, N = a.N, Dreal = a.Dreal, M = a.M, bsz = a.bsz, pad_head = a.pad_head,
              pad_tail = a.pad_tail, qtiles = a.qtiles, kgroups = a.kgroups;
    const float c = a.c;
    // NG > 0: candidate streams with NG block groups (STREAM)
    constexpr bool STREAM = NG > 0;
    using E = Elem<DT>;
    using Sh = ScorePipeShape<D>;
    using SW = FtaSwz<Sh::QSEG>;
    constexpr int KS = D / 16;
    constexpr int QSEG = Sh::QSEG, LQ = Sh::LQ, NBUF = Sh::NBUF;
    __shared__ __align__(1024) unsigned char sK[NBUF][Sh::BUF_B];
    static_assert(GT == 2 || GT == 4, "group top-2 or top-4");
    static_assert(!GH || GT == 4, "fp16 group state holds four keys");
    static_assert(SB == 1 || SB == 2, "blocks of 64 or 128 keys");
    constexpr int GB = GT * (GH ? 2 : 4);  // bytes per (group, query)
    using GRaw = typename GroupRaw<GB>::type;
    __shared__ __align__(16) GRaw sG[STREAM ? NG : 1][256];

    const int bh = wg / qtiles;
    const int qt = wg - bh * qtiles;
    const int b = bh / H, h = bh - (bh / H) * H;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int hf = lane >> 5;
    const int qbase = qt * 256 + wave * 64;
    const uint16_t* qp = q + b * q_sb + h * q_sh;
    const uint16_t* kp = k + b * k_sb + h * k_sh;

    uint4 qf[2][KS];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        const int qi = qbase + t * 32 + (lane & 31);
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            const int d = ks * 16 + hf * 8;
            qf[t][ks] = (qi < N && d < Dreal) ? *reinterpret_cast<const uint4*>(qp + (int64_t)qi * q_sn + d)
                                              : fta_zero4();
        }
    }
    // complete the register loads before the DMA stream (the compiler does not see the DMAs)
    fta_wait_vmcnt<0>();

    // Per-lane DMA sources within a K block: instruction i of this wave fills the
    // 1 KB LDS block i * 4 + wave; roff = (row * k_sn + column) * 2 bytes.
    uint32_t roff[LQ];
#pragma unroll
    for (int i = 0; i < LQ; ++i) {
        const int sidx = (i * 4 + wave) * 64 + lane;
        const int row = sidx / QSEG;
        int j = SW::slot(row, sidx - row * QSEG);
        if (j * 8 >= Dreal) j = 0;  // columns past D meet zero q columns
        roff[i] = (uint32_t)(row * (int)k_sn + j * 8) * 2u;
    }
    const uint32_t lds0 = fta_lds_addr(&sK[0][0]);
    const int U = M * SB;  // 64-key chunks
    auto issue = [&](int u) {
        const uint32_t sb = lds0 + (u & (NBUF - 1)) * Sh::BUF_B;
        const int kb = u * 64 - pad_head;
        if (kb >= 0 && kb + 64 <= N) {
            const uint16_t* base = kp + (int64_t)kb * k_sn;
#pragma unroll
            for (int i = 0; i < LQ; ++i) fta_dma16_so(base, roff[i], sb + (i * 4 + wave) * 1024);
        } else {  // block at a sequence edge: clamp rows (masked to -inf below)
            // addresses formed here, not kept live across the loop for this rare case
            int ln = lane;
            asm volatile("" : "+v"(ln));
#pragma unroll
            for (int i = 0; i < LQ; ++i) {
                const int sidx = (i * 4 + wave) * 64 + ln;
                const int row = sidx / QSEG;
                int j = SW::slot(row, sidx - row * QSEG);
                if (j * 8 >= Dreal) j = 0;
                const int t = min(max(kb + row, 0), N - 1);
                fta_dma16_at(kp + (int64_t)t * k_sn + j * 8, sb + (i * 4 + wave) * 1024);
            }
        }
    };
    // scores of keys 32 s .. 32 s + 31 of a chunk for both query tiles
    auto mma_half = [&](int bi, int s, f32x16 (&acc)[2]) {
        const uint16_t* base = reinterpret_cast<const uint16_t*>(&sK[bi][0]) + s * 32 * QSEG * 8;
        const f32x16 zacc = {};
        uint4 a[KS];
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) a[ks] = *reinterpret_cast<const uint4*>(base + SW::off(lane & 31, 2 * ks + hf));
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            acc[0] = E::mma(a[ks], qf[0][ks], ks ? acc[0] : zacc);
            acc[1] = E::mma(a[ks], qf[1][ks], ks ? acc[1] : zacc);
        }
    };
    auto edge_mask = [&](int u, int s, f32x16 (&acc)[2]) {
        const int kb = u * 64 - pad_head;
        if (kb < 0 || kb + 64 > N) {
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int t = kb + s * 32 + c_row(i, lane);
                if (t < 0 || t >= N) {
                    acc[0][i] = -FTA_INF;
                    acc[1][i] = -FTA_INF;
                }
            }
        }
    };
    auto sums16 = [&](const f32x16 (&acc)[2], const float* Rr, float* e) {
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            float v[16];
#pragma unroll
            for (int i = 0; i < 16; ++i) v[i] = acc[t][i];
            e[t] = fta_sum_exp2<16>(v, c, Rr[t]);
        }
    };
    // R[t]: reference of tile t's query (lane & 31), used by this lane's exps of both
    // tiles; L: running total of the lane's own (tile lane >> 5, query lane & 31)
    float R[2] = {-FTA_INF, -FTA_INF}, L = 0.f;
    const bool own1 = lane >= 32;
    float Rown = -FTA_INF;  // R of the lane's own tile (R[lane >> 5])
    // One pipeline stage, written in issue order: the MFMAs of half s of block mb
    // (into dst) interleaved with the exps of src, 32 / KS exps after each MFMA
    // pair.  The sums use the same 16-term tree as fta_sum_exp2<16>.
    // The order is pinned with empty volatile asm statements (kept in program
    // order by the compiler): group g's K fragment and a scalar copy of the
    // scale used by its exps pass through one, and its exp / add results feed
    // the next group's, so each group's MFMAs, exps and adds stay in their window.
    auto stage = [&](int bi, int s, f32x16 (&dst)[2], const f32x16 (&src)[2], float* e_out) {
        const uint16_t* base = reinterpret_cast<const uint16_t*>(&sK[bi][0]) + s * 32 * QSEG * 8;
        const f32x16 zacc = {};
        uint4 a[KS];
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) a[ks] = *reinterpret_cast<const uint4*>(base + SW::off(lane & 31, 2 * ks + hf));
        constexpr int PER = 32 / KS;
        float ex[2][16];
#pragma unroll
        for (int g = 0; g < KS; ++g) {
            typedef unsigned int u32x4v __attribute__((ext_vector_type(4)));
            u32x4v agv = __builtin_bit_cast(u32x4v, a[g]);
            float cg = c;  // a scalar copy: the group's exps depend on it
            asm volatile("" : "+v"(agv), "+s"(cg));
            const uint4 ag = __builtin_bit_cast(uint4, agv);
            dst[0] = E::mma(ag, qf[0][g], g ? dst[0] : zacc);
            dst[1] = E::mma(ag, qf[1][g], g ? dst[1] : zacc);
#pragma unroll
            for (int u = 0; u < PER; ++u) {
                const int idx = g * PER + u, t = idx >> 4, i = idx & 15;
                ex[t][i] = fta_exp2(fmaf(src[t][i], cg, -R[t]));
            }
            // tree adds whose subtree is complete after this group (same tree and
            // order as fta_sum_exp2<16>: level w adds e[i] += e[i + w], i % 2w == 0)
#pragma unroll
            for (int t = 0; t < 2; ++t)
#pragma unroll
                for (int w = 1; w < 16; w <<= 1)
#pragma unroll
                    for (int i = 0; i + w < 16; i += 2 * w)
                        if ((t * 16 + i + 2 * w - 1) / PER == g) {
                            ex[t][i] += ex[t][i + w];
                            asm volatile("" ::"v"(ex[t][i]));
                        }
#pragma unroll
            for (int u = 0; u < PER; ++u) {
                const int idx = g * PER + u, t = idx >> 4, i = idx & 15;
                if (i & 1) asm volatile("" ::"v"(ex[t][i]));  // odd leaves are consumed by level-1 adds
            }
        }
        e_out[0] = ex[0][0];
        e_out[1] = ex[1][0];
    };

    float gkey = -FTA_INF, tkey = FTA_INF;
    int gidx = 0, tidx = 0, curg = -1, next_start = 0;
    const float adj_head = (pad_head > 0) ? fta_log2((float)bsz / (float)(bsz - pad_head)) : 0.f;
    const float adj_tail = (pad_tail > 0) ? fta_log2((float)bsz / (float)(bsz - pad_tail)) : 0.f;

    // the GT keys of a group-state entry, descending
    auto gdecode = [&](const GRaw& r, float (&t)[GT]) {
        if constexpr (GH) {
            const uint2 u = __builtin_bit_cast(uint2, r);
            t[0] = fta_h2f(u.x);
            t[1] = fta_h2f(u.x >> 16);
            t[2] = fta_h2f(u.y);
            t[3] = fta_h2f(u.y >> 16);
        } else {
            const auto f = __builtin_bit_cast(typename std::conditional<GT == 2, float2, float4>::type, r);
            t[0] = f.x;
            t[1] = f.y;
            if constexpr (GT == 4) {
                t[2] = f.z;
                t[3] = f.w;
            }
        }
    };
    auto gencode = [&](const float (&t)[GT]) -> GRaw {
        if constexpr (GH) {
            return __builtin_bit_cast(GRaw, make_uint2(fta_f2h2(t[0], t[1]), fta_f2h2(t[2], t[3])));
        } else if constexpr (GT == 2) {
            return __builtin_bit_cast(GRaw, make_float2(t[0], t[1]));
        } else {
            return __builtin_bit_cast(GRaw, make_float4(t[0], t[1], t[2], t[3]));
        }
    };
    // the smallest kept key of group j (the bound's operand)
    auto glast = [&](int j) -> float {
        const GRaw r = sG[j][tid];
        if constexpr (GH) {
            return fta_h2f(__builtin_bit_cast(uint2, r).y >> 16);
        } else {
            float t[GT];
            gdecode(r, t);
            return t[GT - 1];
        }
    };
    // fp16 group state holds keys relative to the query's first block key gref,
    // so its 2^-11 relative rounding scales with key differences, not with key
    // magnitudes (near-uniform rows would otherwise pass every block).
    float gref = 0.f;
    // absolute bound from a min over the groups' keys: fp16 keys may sit 2^-11
    // relative above the key they hold, so their bound is lowered by a further
    // 2^-10 relative, and by 2^-22 |gref| for the fp32 add of the reference
    auto gabs = [&](float bnd) -> float {
        return GH ? gref + bnd - (fabsf(bnd) * 0x1p-10f + fabsf(gref) * 0x1p-22f) : bnd;
    };
    auto gmargin = [&](float bnd) -> float { return fta_stream_margin(gabs(bnd)); };

    // candidate-stream state: the wave's current chunk and position in it, its
    // chunk count and entry count, and the current filter bound
    uint2* cst = nullptr;
    int cpos = 0, nch = 1, spos = 0;
    const int64_t sw = (int64_t)wg * 4 + wave;
    // lanes past N never pass: their bound is +inf
    const bool lane_ok = qbase + lane < N;
    float sbnd = lane_ok ? -FTA_INF : FTA_INF;
    if constexpr (STREAM) {
        cst = a.pool + sw * kStreamChunk;
        float ninf[GT];
#pragma unroll
        for (int i = 0; i < GT; ++i) ninf[i] = -FTA_INF;
#pragma unroll
        for (int j = 0; j < NG; ++j) sG[j][tid] = gencode(ninf);
    }

#pragma unroll
    for (int j = 0; j < NBUF - 1; ++j)
        if (j < U) issue(j);
    if (U >= 3)
        fta_wait_vmcnt<2 * LQ>();
    else if (U == 2)
        fta_wait_vmcnt<LQ>();
    else
        fta_wait_vmcnt<0>();
    __syncthreads();
    f32x16 h0[2], h1[2];
    mma_half(0, 0, h0);

    // Chunk u of block m = u / SB; ju = u mod 4 (a compile-time constant in the
    // unrolled main loop, so the K buffer (u mod 4), the sub-chunk (u mod SB) and,
    // for SB = 1, the group slot (m mod NG) become immediates instead of per-read
    // address arithmetic).  bsum carries the block's earlier chunk totals (SB = 2).
    // `interior`: chunk u lies inside the sequence, its block is neither the first
    // nor the last (no head / tail adjustment) and a next chunk exists.
    float bsum = 0.f;
    auto block = [&](int u, auto ju, auto interior) {
        constexpr bool IN = decltype(interior)::value;
        const int bm = int(ju) & (NBUF - 1), bn = (int(ju) + 1) & (NBUF - 1);  // buffers of u, u + 1
        const int m = (SB == 1) ? u : (u >> 1);
        const int sub = (SB == 1) ? 0 : (int(ju) & 1);
        const bool blast = sub == SB - 1;  // the block's last chunk: its value is formed here
        const int gslot = m & (NG > 0 ? NG - 1 : 0);
        // chunk u + 1 resident: chunks issued so far = min(U, u + 3)
        if (IN || u + 1 < U) {
            if (u + 3 <= U)
                fta_wait_vmcnt<LQ>();
            else
                fta_wait_vmcnt<0>();
        }
        __syncthreads();  // chunk u + 1 visible; every wave is past chunk u - 1
        if (u + 3 < U) issue(u + 3);
        // this block's group top-2 entry, read now so its latency hides under the stages
        GRaw gtop = {};
        if constexpr (STREAM)
            if (blast) gtop = sG[gslot][tid];

        float e0[2], e1[2];
        const int kb = u * 64 - pad_head;
        if (IN || u + 1 < U) {
            // Every block but the last runs the same two stages; a block at a
            // sequence edge first masks its scores in place (uniform branches),
            // so the loop-carried accumulators have one definition and keep
            // their registers.  Masked scores are -inf: their exps are 0.
            // pad_head, pad_tail < b and b | pad_head + N + pad_tail (checked on the host):
            // only the chunks of the first and the last block can reach past the sequence
            const bool edge = !IN && (kb < 0 || kb + 64 > N);
            if (edge) edge_mask(u, 0, h0);
            stage(bm, 1, h1, h0, e0);     // MFMAs of half 1 of chunk u, exps of half 0
            if (edge) edge_mask(u, 1, h1);
            stage(bn, 0, h0, h1, e1);     // MFMAs of half 0 of chunk u + 1, exps of half 1
        } else {
            edge_mask(u, 0, h0);
            mma_half(bm, 1, h1);
            sums16(h0, R, e0);
            edge_mask(u, 1, h1);
            if (u + 1 < U) {
                mma_half(bn, 0, h0);
            }
            sums16(h1, R, e1);
        }
        // chunk total of the lane's own (tile, query): lanes l and l ^ 32 hold halves
        // of each query's sum; one lane-half swap adds them (the same operand pairs as
        // part + part[l ^ 32], so the results are identical)
        float tot_own;
        {
            float a = e0[0] + e1[0], b = e0[1] + e1[1];
            fta_swap32(a, b);
            tot_own = a + b;
        }
        // every (tile, query) is owned by one lane, so wave votes on tot_own cover both
        // tiles.  The rare cases (a total that overflows the reference, or grows
        // large) are handled around the common update, so R and L keep one
        // definition on the common path (no register copies at the merges).
        const bool rare = __ballot(!(tot_own <= 0x1p40f)) != 0ull;  // large, infinite or NaN
        {
            if (rare && __ballot(!(tot_own < 0x1p100f)) != 0ull) {
                // exact path: reference = this block's max (scores recomputed from LDS)
                f32x16 x0[2], x1[2];
                mma_half(bm, 0, x0);
                mma_half(bm, 1, x1);
                edge_mask(u, 0, x0);
                edge_mask(u, 1, x1);
                const float R_old = own1 ? R[1] : R[0];
#pragma unroll
                for (int t = 0; t < 2; ++t) {
                    float mx = x0[t][0];
#pragma unroll
                    for (int i = 1; i < 16; ++i) mx = fmaxf(mx, x0[t][i]);
#pragma unroll
                    for (int i = 0; i < 16; ++i) mx = fmaxf(mx, x1[t][i]);
                    mx = fmaxf(mx, fta_xor32(mx));
                    R[t] = (mx == -FTA_INF) ? 0.f : mx * c;
                }
                const float R_new = own1 ? R[1] : R[0];
                Rown = R_new;
                L = (L > 0.f) ? L * fta_exp2(R_old - R_new) : 0.f;
                if constexpr (SB > 1) bsum = (bsum > 0.f) ? bsum * fta_exp2(R_old - R_new) : 0.f;
                float f0[2], f1[2];
                sums16(x0, R, f0);
                sums16(x1, R, f1);
                float tot[2];
#pragma unroll
                for (int t = 0; t < 2; ++t) {
                    const float part = f0[t] + f1[t];
                    tot[t] = part + fta_xor32(part);
                }
                tot_own = own1 ? tot[1] : tot[0];
            }
        }
        // block total so far (the chunks before this one were rescaled with R)
        float bs = tot_own;
        if constexpr (SB > 1) bs = sub ? bsum + tot_own : tot_own;
        // only the lane's own block lse is stored (log2(0) = -inf)
        const float mine = Rown + fta_log2(bs);
        L += tot_own;
        {
            if (rare && __ballot(bs > 0x1p40f) != 0ull) {
                // rebase a large total on this block's lse (both tiles' references,
                // so this lane's exps of the other tile stay in step with its owner)
                float x = bs, y = bs;
                fta_swap32(x, y);
                const float other = own1 ? x : y;
                const float tot[2] = {own1 ? other : bs, own1 ? bs : other};
#pragma unroll
                for (int t = 0; t < 2; ++t)
                    if (tot[t] > 0x1p40f) {
                        const float Rn = R[t] + fta_log2(tot[t]);
                        if ((t == 1) == own1) {
                            const float f = fta_exp2(R[t] - Rn);
                            L *= f;
                            if constexpr (SB > 1) bs *= f;
                        }
                        R[t] = Rn;
                    }
                Rown = own1 ? R[1] : R[0];
            }
        }
        if constexpr (SB > 1) bsum = bs;
        if (!blast) return;
        const int qi = qbase + lane;
        if constexpr (STREAM) {
            // wave-uniform adjustment and edge flag (partial edge blocks always pass)
            const float adj = IN ? 0.f : ((m == 0) ? adj_head : 0.f) + ((m == M - 1) ? adj_tail : 0.f);
            const bool em = !IN && (((m == 0) & (pad_head > 0)) | ((m == M - 1) & (pad_tail > 0)));
            const float ak = IN ? mine : mine + adj;
            const bool pass = (ak >= sbnd) | (em & lane_ok);
            const unsigned long long mk = __ballot(pass);
            const int rank = __builtin_amdgcn_mbcnt_hi((uint32_t)(mk >> 32),
                                                       __builtin_amdgcn_mbcnt_lo((uint32_t)mk, 0u));
            const int nmk = __popcll(mk);
            const uint2 entry = make_uint2(__builtin_bit_cast(uint32_t, mine), ((uint32_t)lane << 16) | m);
            if (cpos + nmk <= kStreamChunk) {
                if (pass) {  // wave-uniform base, 32-bit lane offset
                    uint2* dst = cst + cpos;
                    dst[(uint32_t)rank] = entry;
                }
                cpos += nmk;
            } else {
                // the chunk is full (or the pool ran out before: cpos is then past
                // any chunk): continue in a new chunk from the pool
                int id = 0;
                if (lane == 0 && cpos <= kStreamChunk) id = atomicAdd(a.pool_ctr, 1);
                id = __builtin_amdgcn_readfirstlane(id) + a.total * 4;
                if (cpos > kStreamChunk || id >= a.pool_chunks || nch >= a.maxch) {
                    cpos = 0x40000000;  // out of pool: no further entries are stored
                } else {
                    if (lane == 0) a.chunk_tab[sw * a.maxch + nch] = id;
                    ++nch;
                    uint2* nxt = a.pool + (int64_t)id * kStreamChunk;
                    const int room = kStreamChunk - cpos;
                    if (pass) {
                        uint2* dst = (rank < room) ? cst + cpos + rank : nxt + (rank - room);
                        *dst = entry;
                    }
                    cst = nxt;
                    cpos += nmk - kStreamChunk;
                }
            }
            spos += nmk;
            // group top-GT insertion (t descending): new t0 = max(t0, ak), new t_i =
            // med3(t_{i-1}, t_i, ak).  Written as instructions: the compiler's max /
            // med3 first quiet every operand, and no value here is a NaN.  fp16 state
            // takes ak - gref clamped to the largest finite half (below the key).
            float t[GT], nt[GT];
            gdecode(gtop, t);
            float akg = ak;
            if constexpr (GH) {
                if (!IN && m == 0) gref = (fabsf(ak) < FTA_INF) ? ak : 0.f;
                asm("v_min_f32 %0, %1, %2" : "=v"(akg) : "v"(ak - gref), "v"(65504.f));
            }
            asm("v_max_f32 %0, %1, %2" : "=v"(nt[0]) : "v"(t[0]), "v"(akg));
#pragma unroll
            for (int i = 1; i < GT; ++i)
                asm("v_med3_f32 %0, %1, %2, %3" : "=v"(nt[i]) : "v"(t[i - 1]), "v"(t[i]), "v"(akg));
            sG[gslot][tid] = gencode(nt);
            if (gslot == NG - 1) {
                float bnd = glast(0);
#pragma unroll
                for (int j = 1; j < NG; ++j) bnd = __builtin_amdgcn_fmed3f(bnd, glast(j), -FTA_INF);
                sbnd = lane_ok ? gmargin(bnd) : FTA_INF;
            }
        } else {
            if (qi < N) {
                if (a.blk_ld == 0)
                    a.blk_lse[((int64_t)bh * M + m) * N + qi] = mine;
                else
                    a.blk_lse[(int64_t)m * a.blk_ld + (qi - qt * 256)] = mine;
            }
        }
        if (!STREAM && kgroups > 0) {
            float key = mine;
            if (m == 0) key += adj_head;
            if (m == M - 1) key += adj_tail;
            if (m == next_start) {
                if (curg >= 0 && gkey < tkey) {
                    tkey = gkey;
                    tidx = gidx;
                }
                ++curg;
                next_start = ((curg + 1) * M + kgroups - 1) / kgroups;  // first block of group curg + 1
                gkey = key;
                gidx = m;
            } else if (key > gkey) {
                gkey = key;
                gidx = m;
            }
        }
    };
    // every chunk but the last always produces the next chunk's half 0
    {
        using I0 = std::integral_constant<int, 0>;
        using I1 = std::integral_constant<int, 1>;
        using I2 = std::integral_constant<int, 2>;
        using I3 = std::integral_constant<int, 3>;
        if constexpr (SB == 1) {
            int m = 0;
            if (M > 1) {
                block(0, I0{}, std::false_type{});
                m = 1;
            }
            for (; m + 4 < M; m += 4) {  // m = 1 mod 4
                block(m, I1{}, std::true_type{});
                block(m + 1, I2{}, std::true_type{});
                block(m + 2, I3{}, std::true_type{});
                block(m + 3, I0{}, std::true_type{});
            }
            for (; m + 1 < M; ++m) block(m, m & 3, std::true_type{});
            block(M - 1, (M - 1) & 3, std::false_type{});
        } else {
            // the two chunks of the first and of the last block run as edge chunks
            block(0, I0{}, std::false_type{});
            block(1, I1{}, std::false_type{});
            int u = 2;
            for (; u + 4 <= U - 2; u += 4) {  // u = 2 mod 4
                block(u, I2{}, std::true_type{});
                block(u + 1, I3{}, std::true_type{});
                block(u + 2, I0{}, std::true_type{});
                block(u + 3, I1{}, std::true_type{});
            }
            for (; u < U - 2; ++u) block(u, u & 3, std::true_type{});
            if (U > 2) {
                block(U - 2, (U - 2) & 3, std::false_type{});
                block(U - 1, (U - 1) & 3, std::false_type{});
            }
        }
    }

    const int qi = qbase + lane;
    const float rlf = (L > 0.f) ? Rown + fta_log2(L) : -FTA_INF;
    float bnd = -FTA_INF;
    if constexpr (STREAM) {
        bnd = glast(0);
#pragma unroll
        for (int j = 1; j < NG; ++j) bnd = fminf(bnd, glast(j));
        bnd = gabs(bnd);  // fp16 state: relative to gref, lowered by its rounding
        // The filter's margin orders the selector's averages 2^(key - rl) / b only
        // while they are normal fp32 numbers: a final bound more than 100 log2
        // units below the row total (averages that may be subnormal or zero, whose
        // ties fall to the block index) sends the tile to the exact fallback, as
        // an exhausted pool does.
        const bool risky = lane_ok && bnd > -FTA_INF && !(bnd - rlf >= -100.f);
        const bool redo = (cpos > kStreamChunk) || __ballot(risky) != 0ull;
        if (lane == 0) a.count[sw] = redo ? -1 : spos;
    }
    if (qi < N) {
        a.row_lse[(int64_t)bh * N + qi] = rlf;
        if constexpr (STREAM) {
            a.tau_key[(int64_t)bh * N + qi] = bnd;
        } else if (kgroups > 0) {
            if (curg >= 0 && gkey < tkey) tidx = gidx;
            a.tau_idx[(int64_t)bh * N + qi] = tidx;
        }
    }
}

template <int DT, int D, int NG, int GT, bool GH, int SB>
__global__ __launch_bounds__(256, 2) void fta_block_score_lse_pipe_kernel(const ScoreArgs a) {
    fta_score_tile<DT, D, NG, GT, GH, SB>(a, fta_xcd_remap(blockIdx.x, a.total));
}

// ----------------------------------------------------------------------------
// Stage 2a: materialise scores[bh][n][m] = 2^{lse2[bh][m][n] - lse2[bh][n]}.
// 64 x 64 tiles transposed through LDS.
// ----------------------------------------------------------------------------
__global__ __launch_bounds__(256) void fta_block_normalize_kernel(const float* __restrict__ blk_lse,
                                                                  const float* __restrict__ row_lse,
                                                                  float* __restrict__ scores, int N, int M,
                                                                  int ntiles_n, int ntiles_m) {
    __shared__ float tile[64][65];
    const int bh = blockIdx.x / (ntiles_n * ntiles_m);
    const int r = blockIdx.x - bh * ntiles_n * ntiles_m;
    const int tn = r / ntiles_m, tm = r - (r / ntiles_m) * ntiles_m;
    const int n0 = tn * 64, m0 = tm * 64;
    const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
    for (int mm = ty; mm < 64; mm += 4) {
        const int m = m0 + mm, n = n0 + tx;
        float v = 0.f;
        if (m < M && n < N) v = blk_lse[((int64_t)bh * M + m) * N + n] - row_lse[(int64_t)bh * N + n];
        tile[mm][tx] = v;
    }
    __syncthreads();
    for (int nn = ty; nn < 64; nn += 4) {
        const int n = n0 + nn, m = m0 + tx;
        if (m < M && n < N) scores[((int64_t)bh * N + n) * M + m] = fta_exp2(tile[tx][nn]);
    }
}

// ----------------------------------------------------------------------------
// Stage 2b: top-k selection, one lane per query row.
// Single pass over the M blocks: a block becomes a candidate when it beats the
// current K-th best (tau); candidates are parked in a per-lane LDS list and
// merged into a sorted register list (insertion network) whenever some lane's
// list is full, after which tau tightens.  Exact for any input; deterministic.
// MODE 0 reads raw scores in[row * stride_row + m * stride_m];
// MODE 1 reads the lse2 intermediate ([BH][M][N]) and row totals.
// ----------------------------------------------------------------------------
// (v, i) ranks above (w, j): larger value, ties to the lower index.  Bitwise
// operators, not && / ||: the short-circuit form compiles to an exec-mask
// branch per comparison inside the insertion network.
__device__ __forceinline__ bool fta_better(float v, int i, float w, int j) {
    return (v > w) | ((v == w) & (i < j));
}

// raw / valid_count with IEEE division; for a power-of-two block size the
// interior blocks' quotient is the (exact) product with 1 / b, which is the
// same correctly rounded value, and the division sequence runs only when some
// lane of the wave holds a partial edge block.
__device__ __forceinline__ float fta_avg(float raw, int vc, int bsz, float inv_b) {
    float a = raw * inv_b;
    const bool slow = (vc != bsz) | (inv_b == 0.f);
    if (__ballot(slow) != 0ull) {
        const float q = raw / (float)vc;
        a = slow ? q : a;
    }
    return a;
}

__device__ __forceinline__ int fta_valid_count(int m, int M, int bsz, int pad_head, int pad_tail) {
    int vc = bsz;
    if (pad_head > 0 && m == 0) vc -= pad_head;
    if (pad_tail > 0 && m == M - 1) vc -= pad_tail;
    return vc;
}

// Merge a lane's parked candidates into its sorted register list, then
// tighten (tv, ti) to the m_out-th entry.  Candidates are parked by a cheap
// pre-filter only (the loaded value x and block m); the exact tests run here,
// for candidates alone: the pre-filter bound (pre) and raw >= thr_norm, both
// waived for partial edge blocks, then avg = raw / valid_count must beat the
// current m_out-th entry.  Bounds only tighten, so testing against the bounds
// at flush time rather than at parking time drops only blocks that could not
// be in the final list.  Insertion network, top down: slot p takes slot p-1's
// entry when the candidate beats it, the candidate when it beats only slot p.
// A function rather than a lambda so that it is always inlined: the register
// lists must never be addressed through memory.
template <int KB, int CAP, int MODE>
__device__ __forceinline__ void fta_topk_flush(float (&lv)[KB], int (&li)[KB], int& cnt, const float (&cv)[CAP][64],
                                               const int (&ci)[CAP][64], int lane, bool active, float rl, float pre,
                                               float thr_norm, int M, int bsz, int pad_head, int pad_tail,
                                               int m_out, float threshold, float& tv, int& ti) {
    // 1 / b when b is a power of two (an exact reciprocal), else 0
    const float inv_b = ((bsz & (bsz - 1)) == 0) ? 1.f / (float)bsz : 0.f;
    int mc = cnt;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) mc = max(mc, __shfl_xor(mc, off, 64));
    if constexpr (KB == 32) {
        // Lists of 32: the parked candidates are merged 16 at a time.  The batch
        // is sorted (bitonic, descending by (avg, -index)); the top KB of list +
        // batch is then max(list[i], batch[KB - 1 - i]) (a bitonic sequence:
        // only the last 16 positions compare), sorted by a bitonic merge.  The
        // list ends as the top KB of the accepted candidates, as with one
        // insertion per candidate, at ~11 compare-exchanges per candidate
        // instead of KB insertion steps.  (At KB = 64 the lists and the batch no
        // longer fit the registers of two waves per SIMD: the insertion network
        // below stays.)
        auto ce = [](float& va, int& ia, float& vb, int& ib) {  // the better pair first
            const bool sw = fta_better(vb, ib, va, ia);
            const float v0 = sw ? vb : va, v1 = sw ? va : vb;
            const int i0 = sw ? ib : ia, i1 = sw ? ia : ib;
            va = v0;
            vb = v1;
            ia = i0;
            ib = i1;
        };
        for (int jb = 0; jb < mc; jb += 16) {
            float bv[16];
            int bi[16];
            bool any = false;
#pragma unroll
            for (int u = 0; u < 16; ++u) {
                const int j = jb + u;
                const bool in = (j < cnt) & (j < CAP);
                const float xs = in ? cv[in ? j : 0][lane] : 0.f;
                const int m = in ? ci[in ? j : 0][lane] : 0;
                const bool edge = ((m == 0) & (pad_head > 0)) | ((m == M - 1) & (pad_tail > 0));
                const float x = (MODE == 0) ? xs : xs - rl;
                const float raw = (MODE == 0) ? x : fta_exp2(x);
                const int vc = fta_valid_count(m, M, bsz, pad_head, pad_tail);
                const float avg = fta_avg(raw, vc, bsz, inv_b);
                const bool ok = active & in & (edge | ((x >= pre) & (raw >= thr_norm))) & fta_better(avg, m, tv, ti);
                bv[u] = ok ? avg : -FTA_INF;
                bi[u] = ok ? m : 0x7fffffff;
                any |= ok;
            }
            if (__ballot(any) == 0ull) continue;
#pragma unroll
            for (int k = 2; k <= 16; k <<= 1)
#pragma unroll
                for (int j = k >> 1; j > 0; j >>= 1)
#pragma unroll
                    for (int i = 0; i < 16; ++i) {
                        const int l = i ^ j;
                        if (l > i) {
                            if ((i & k) == 0)
                                ce(bv[i], bi[i], bv[l], bi[l]);
                            else
                                ce(bv[l], bi[l], bv[i], bi[i]);
                        }
                    }
#pragma unroll
            for (int i = KB - 16; i < KB; ++i) {
                const float v2 = bv[KB - 1 - i];
                const int i2 = bi[KB - 1 - i];
                const bool take = fta_better(v2, i2, lv[i], li[i]);
                lv[i] = take ? v2 : lv[i];
                li[i] = take ? i2 : li[i];
            }
#pragma unroll
            for (int j = KB >> 1; j > 0; j >>= 1)
#pragma unroll
                for (int i = 0; i < KB; ++i)
                    if ((i & j) == 0) ce(lv[i], li[i], lv[i + j], li[i + j]);
#pragma unroll
            for (int p = 0; p < KB; ++p)
                if (p == m_out - 1 && li[p] != 0x7fffffff) {
                    tv = lv[p];
                    ti = li[p];
                }
        }
        mc = 0;  // the per-candidate loop below has nothing left
    }
    for (int j = 0; j < mc; ++j) {
        const float xs = cv[j][lane];
        const int m = ci[j][lane];
        const bool edge = ((m == 0) & (pad_head > 0)) | ((m == M - 1) & (pad_tail > 0));
        const float x = (MODE == 0) ? xs : xs - rl;
        const float raw = (MODE == 0) ? x : fta_exp2(x);
        const int vc = fta_valid_count(m, M, bsz, pad_head, pad_tail);
        const float avg = fta_avg(raw, vc, bsz, inv_b);
        const bool ok = active & (j < cnt) & (edge | ((x >= pre) & (raw >= thr_norm))) &
                        fta_better(avg, m, tv, ti);
        if (__ballot(ok) == 0ull) continue;  // no lane inserts: skip the network
        const float v = ok ? avg : -FTA_INF;
        const int id = ok ? m : 0x7fffffff;
        bool bhi = fta_better(v, id, lv[KB - 1], li[KB - 1]);
#pragma unroll
        for (int p = KB - 1; p > 0; --p) {
            const bool blo = fta_better(v, id, lv[p - 1], li[p - 1]);
            const float nv = blo ? lv[p - 1] : (bhi ? v : lv[p]);
            const int ni = blo ? li[p - 1] : (bhi ? id : li[p]);
            lv[p] = nv;
            li[p] = ni;
            bhi = blo;
        }
        if (bhi) {
            lv[0] = v;
            li[0] = id;
        }
        if (m_out == KB && li[KB - 1] != 0x7fffffff) {  // a full list bounds the rest of the flush
            tv = lv[KB - 1];
            ti = li[KB - 1];
        }
    }
    cnt = 0;
#pragma unroll
    for (int p = 0; p < KB; ++p)
        if (p == m_out - 1 && li[p] != 0x7fffffff) {
            tv = lv[p];
            ti = li[p];
        }
    // Threshold cut of the current list.  Later candidates only raise each
    // prefix sum of the sorted raw values (the i-th largest of a superset is at
    // least the i-th largest of the set, and fp32 rounding is monotone), so the
    // final cut is at or before the current one, and a block ranked below the
    // current cut entry is never output: that entry bounds the rest.
    float cs = 0.f;
    bool found = false;
#pragma unroll
    for (int p = 0; p < KB; ++p) {
        const bool use = (p < m_out) & !found & (li[p] != 0x7fffffff);
        const float rw = __fmul_rn(lv[p], (float)fta_valid_count(li[p], M, bsz, pad_head, pad_tail));
        cs = use ? __fadd_rn(cs, rw) : cs;
        const bool hit = use & (cs >= threshold);
        if (hit & fta_better(lv[p], li[p], tv, ti)) {
            tv = lv[p];
            ti = li[p];
        }
        found = found | hit;
    }
}

// Threshold cut and output of a wave's sorted register lists (rows wrow0 ..
// wrow0 + nrows - 1, lane = row - wrow0): keep positions up to the first whose
// sequential fp32 cumulative raw score reaches the threshold, -1 / 0 after.
// Outputs are staged in the wave's LDS buffer `st` when every list fits.
template <int KB, int CAP>
__device__ __forceinline__ void fta_topk_emit(float (&lv)[KB], int (&li)[KB], int m_out, int M, int bsz,
                                              int pad_head, int pad_tail, float threshold,
                                              int32_t* __restrict__ out_idx, float* __restrict__ out_raw,
                                              float* __restrict__ out_avg, int64_t wrow0, int nrows, int lane,
                                              bool active, int64_t row, float (&stage)[CAP][64]) {
    float cs = 0.f;
    int cut = m_out;
    bool found = false;
#pragma unroll
    for (int p = 0; p < KB; ++p) {
        if (p < m_out && !found) {
            const float rw = __fmul_rn(lv[p], (float)fta_valid_count(li[p], M, bsz, pad_head, pad_tail));
            cs = __fadd_rn(cs, rw);
            if (cs >= threshold) {
                cut = p + 1;
                found = true;
            }
        }
    }
    float rawv[KB];
#pragma unroll
    for (int p = 0; p < KB; ++p) {
        const bool keep = p < cut;
        rawv[p] = keep ? __fmul_rn(lv[p], (float)fta_valid_count(li[p], M, bsz, pad_head, pad_tail)) : 0.f;
        lv[p] = keep ? lv[p] : 0.f;
        li[p] = keep ? li[p] : -1;
    }
    const bool aligned = ((reinterpret_cast<uintptr_t>(out_idx) | reinterpret_cast<uintptr_t>(out_raw) |
                           reinterpret_cast<uintptr_t>(out_avg)) & 15) == 0;
    if (aligned) {
        // Stage each output's rows x m_out block (contiguous in HBM) in this wave's
        // candidate buffer, then write it with 16-byte stores over consecutive
        // addresses instead of one 4-byte store per (lane, slot), which for
        // m_out = 32 / 64 touched 64 cache lines per store.  Rows go in passes
        // of rpp (a multiple of 4, so every pass starts 16-byte aligned) that
        // fit the CAP x 64 buffer.
        float* st = &stage[0][0];
        const int rpp = min(64, ((CAP * 64) / m_out) & ~3);
#pragma unroll
        for (int k = 0; k < 3; ++k) {
            float* out = (k == 0) ? reinterpret_cast<float*>(out_idx) : (k == 1) ? out_raw : out_avg;
            for (int r0 = 0; r0 < nrows; r0 += rpp) {
                const int rn = min(rpp, nrows - r0);
                if (lane >= r0 && lane < r0 + rn) {
#pragma unroll
                    for (int p = 0; p < KB; ++p)
                        if (p < m_out)
                            st[(lane - r0) * m_out + p] =
                                (k == 0) ? __builtin_bit_cast(float, li[p]) : (k == 1) ? rawv[p] : lv[p];
                }
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                float* o = out + (wrow0 + r0) * m_out;
                const int total = rn * m_out, n4 = total >> 2;
                for (int c = lane; c < n4; c += 64)
                    reinterpret_cast<float4*>(o)[c] = reinterpret_cast<const float4*>(st)[c];
                for (int e = (n4 << 2) + lane; e < total; e += 64) o[e] = st[e];
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            }
        }
        return;
    }
    if (!active) return;
    const int64_t o = (int64_t)row * m_out;
#pragma unroll
    for (int p = 0; p < KB; ++p) {
        if (p < m_out) {
            out_idx[o + p] = li[p];
            out_avg[o + p] = lv[p];
            out_raw[o + p] = rawv[p];
        }
    }
}

// Rows blk * 256 .. blk * 256 + 255 of the selection (one row per thread).
template <int KB, int MODE>
__device__ __forceinline__ void fta_topk_rows(
    const float* __restrict__ in, int64_t stride_row, int64_t stride_m, const float* __restrict__ row_lse,
    int N, int rows, int M, int m_out, int bsz, int pad_head, int pad_tail, float threshold,
    int32_t* __restrict__ out_idx, float* __restrict__ out_raw, float* __restrict__ out_avg,
    const int32_t* __restrict__ tau_idx, const int blk) {
    constexpr int LDB = 24;             // blocks loaded per batch
    constexpr int UNR = 8;              // blocks tested between candidate-list checks
    constexpr int CAP = 12 + UNR;       // a sub-batch starts with at most CAP - UNR parked candidates
    __shared__ __align__(16) float cand_v[4][CAP][64];
    __shared__ int cand_i[4][CAP][64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int row = blk * 256 + tid;
    const bool active = row < rows;

    float lv[KB];
    int li[KB];
#pragma unroll
    for (int p = 0; p < KB; ++p) {
        lv[p] = -FTA_INF;
        li[p] = 0x7fffffff;
    }
    float tv = -FTA_INF;
    int ti = 0x7fffffff;
    int cnt = 0;

    const float* src = nullptr;
    float rl = 0.f;
    int64_t bh = 0, n = 0;
    if (MODE == 0) {
        src = in + (int64_t)(active ? row : 0) * stride_row;
    } else {
        bh = (active ? row : 0) / N;
        n = (active ? row : 0) - bh * N;
        src = in + bh * (int64_t)M * N + n;
        rl = row_lse[active ? row : 0];
    }

    // Raw-score pre-filter: a block can only beat tau if raw >= tau * vc; the
    // bound is relaxed by 2^-20 relative so that the exact (avg, index) test
    // below decides every candidate.
    float thr_norm = -FTA_INF;
    // MODE 1 tests x = lse2 - row_lse2 against log2(thr_norm) instead of
    // 2^x >= thr_norm, with a 2^-12 margin far above exp2 / log2 rounding, so
    // the test stays conservative and exp2 runs only for candidates.
    float thr_log = -FTA_INF;
    auto set_thr = [&] __attribute__((always_inline)) () {
        const float t = tv * (float)bsz;
        thr_norm = t - fabsf(t) * 9.5367431640625e-07f;
        thr_log = (thr_norm > 0.f) ? fta_log2(thr_norm) - 2.44140625e-04f : -FTA_INF;
    };
    if (MODE == 1 && tau_idx != nullptr && active) {
        const int t0 = tau_idx[row];
        const float rt = fta_exp2(src[(int64_t)t0 * N] - rl);
        const float at = rt / (float)fta_valid_count(t0, M, bsz, pad_head, pad_tail);
        tv = at - fabsf(at) * 1.52587890625e-05f;  // at least m_out blocks have avg >= this
        ti = 0x7fffffff;
    }
    set_thr();


    // Unconditional loads (an inactive lane reads row 0), clamped past M, two
    // batches in flight: batch k + 1 loads while batch k is tested.
    auto load_batch = [&] __attribute__((always_inline)) (int m1, float (&xs)[LDB]) {
#pragma unroll
        for (int u = 0; u < LDB; ++u) {
            const int m = min(m1 + u, M - 1);
            xs[u] = (MODE == 0) ? src[m * stride_m] : src[(int64_t)m * N];
        }
    };
    // Scan: every block of a sub-batch is parked at slot cnt of the lane's list
    // and cnt advances when the pre-filter passes (x >= pre, or a partial edge
    // block), with no branch per block: the lanes of a wave find candidates at
    // unrelated blocks, so a per-block branch would run for almost every block.
    auto flush = [&] __attribute__((always_inline)) () {
        fta_topk_flush<KB, CAP, MODE>(lv, li, cnt, cand_v[wave], cand_i[wave], lane, active, rl,
                                      (MODE == 0) ? thr_norm : thr_log, thr_norm, M, bsz, pad_head, pad_tail,
                                      m_out, threshold, tv, ti);
        set_thr();
    };
    auto test_batch = [&] __attribute__((always_inline)) (int m1, const float (&xs)[LDB]) {
        const bool edges = (m1 == 0 && pad_head > 0) || (m1 + LDB >= M && pad_tail > 0);
        // the lane's pre-filter bound; +inf parks nothing for lanes past the last row
        const float pre = active ? ((MODE == 0) ? thr_norm : thr_log) : FTA_INF;
        const float pre_edge = active ? -FTA_INF : FTA_INF;  // edge blocks: parked unconditionally
        // Skip the batch when no lane can park a block of it: the largest value
        // of each lane's batch is below its bound and the batch holds no edge
        // block.  Exact: the scan below would park nothing.
        {
            float bm = xs[0];
#pragma unroll
            for (int u = 1; u < LDB; ++u) bm = fmaxf(bm, xs[u]);
            const float bx = (MODE == 0) ? bm : bm - rl;
            if (!edges && __ballot(bx >= pre) == 0ull) return;
        }
#pragma unroll
        for (int sb = 0; sb < LDB; sb += UNR) {
            if (m1 + sb >= M) break;
#pragma unroll
            for (int u = 0; u < UNR; ++u) {
                const int m = m1 + sb + u;
                const float x = (MODE == 0) ? xs[sb + u] : xs[sb + u] - rl;
                // per-block bound, selected by wave-uniform conditions (no branch)
                const bool em = edges && ((m == 0 && pad_head > 0) || (m == M - 1 && pad_tail > 0));
                const float pm = (m >= M) ? FTA_INF : (em ? pre_edge : pre);
                const bool pass = x >= pm;
                cand_v[wave][cnt][lane] = xs[sb + u];
                cand_i[wave][cnt][lane] = m;
                cnt += pass ? 1 : 0;
            }
            if (__ballot(cnt > CAP - UNR) != 0ull) flush();
        }
    };
    float xa[LDB], xb[LDB];
    load_batch(0, xa);
    for (int m1 = 0; m1 < M; m1 += 2 * LDB) {
        load_batch(m1 + LDB, xb);  // clamped: a batch past M rereads block M - 1
        test_batch(m1, xa);
        if (m1 + LDB >= M) break;
        load_batch(m1 + 2 * LDB, xa);
        test_batch(m1 + LDB, xb);
    }
    flush();

    // the wave's rows are consecutive: rows wrow0 .. wrow0 + nrows - 1
    const int64_t wrow0 = (int64_t)blk * 256 + wave * 64;
    const int nrows = (int)min((int64_t)64, (int64_t)rows - wrow0);
    if (nrows <= 0) return;
    fta_topk_emit<KB, CAP>(lv, li, m_out, M, bsz, pad_head, pad_tail, threshold, out_idx, out_raw, out_avg, wrow0,
                           nrows, lane, active, row, cand_v[wave]);
}

// Lists of <= 16 entries fit 4 waves per SIMD (<= 128 VGPRs), which keeps more
// of the scan's loads in flight; longer lists run at 2 waves per SIMD (a
// 64-entry list then spills a few registers, still 40% faster than 1 wave).
template <int KB, int MODE>
__global__ __launch_bounds__(256, (KB <= 16) ? 4 : 2) void fta_topk_select_kernel(
    const float* __restrict__ in, int64_t stride_row, int64_t stride_m, const float* __restrict__ row_lse,
    int N, int rows, int M, int m_out, int bsz, int pad_head, int pad_tail, float threshold,
    int32_t* __restrict__ out_idx, float* __restrict__ out_raw, float* __restrict__ out_avg,
    const int32_t* __restrict__ tau_idx) {
    fta_topk_rows<KB, MODE>(in, stride_row, stride_m, row_lse, N, rows, M, m_out, bsz, pad_head, pad_tail,
                            threshold, out_idx, out_raw, out_avg, tau_idx, blockIdx.x);
}

// Top-k selection over the candidate streams of the pipelined scoring kernel
// (STREAM = true).  One wave per scoring wave (64 consecutive queries of one
// b*h, lane = query); the workgroup's 4 waves are one scoring workgroup's.
// The wave reads its stream 64 entries at a time (coalesced), and each entry
// that passes its owner's pre-filter (value >= the owner's bound, kept in LDS
// in the value domain) is parked in the owner's LDS candidate list at a slot
// taken with an LDS atomic.  When an entry finds its owner's list full, every
// lane merges its parked candidates (fta_topk_flush: exact tests and the
// insertion network) and the entry is parked again.  Each owner's bound starts
// from tau_key (at least m_out blocks rank at or above it) and tightens as its
// list fills.
//
// The streams are chains of kStreamChunk-entry chunks (ScoreArgs).  A tile
// (workgroup) with a wave whose stream ran out of pool (count -1) selects
// nothing: it appends its tile index to ovf_list (count in *ovf_cnt) for the
// fallback kernel, which scores and selects those tiles again.
template <int KB>
__global__ __launch_bounds__(256, (KB <= 16) ? 4 : 2) void fta_topk_stream_kernel(
    const uint2* __restrict__ pool, const int* __restrict__ cand_count, const int* __restrict__ chunk_tab, int maxch,
    const float* __restrict__ tau_key, const float* __restrict__ row_lse, int N, int qtiles, int M, int m_out,
    int bsz, int pad_head, int pad_tail, float threshold, int32_t* __restrict__ out_idx, float* __restrict__ out_raw,
    float* __restrict__ out_avg, int* __restrict__ ovf_list, int* __restrict__ ovf_cnt, int pool_chunks) {
    constexpr int CAP = 16;
    __shared__ __align__(16) float cand_v[4][CAP][64];
    __shared__ int cand_i[4][CAP][64];
    __shared__ int s_cnt[4][64];
    __shared__ float s_pre[4][64];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int bh = blockIdx.x / qtiles;
    const int n0 = (blockIdx.x - bh * qtiles) * 256 + wave * 64;
    const int n = n0 + lane;
    const bool active = n < N;
    const int64_t row = (int64_t)bh * N + (active ? n : 0);
    const int64_t sw = (int64_t)blockIdx.x * 4 + wave;
    {
        const int* c4 = cand_count + (int64_t)blockIdx.x * 4;
        if (min(min(c4[0], c4[1]), min(c4[2], c4[3])) < 0) {  // a stream of this tile is incomplete
            if (tid == 0) {
                const int k = atomicAdd(ovf_cnt, 1);
                if ((unsigned)k < gridDim.x) ovf_list[k] = blockIdx.x;
            }
            return;
        }
    }
    const int* tab = chunk_tab + sw * maxch;
    // Counts, chunk ids and the fallback count are read back from the workspace;
    // they are clamped to what the workspace holds, so a workspace that no scorer
    // run filled gives undefined outputs but no access outside it.
    const int total = min(__builtin_amdgcn_readfirstlane(cand_count[sw]), maxch * kStreamChunk);

    float lv[KB];
    int li[KB];
#pragma unroll
    for (int p = 0; p < KB; ++p) {
        lv[p] = -FTA_INF;
        li[p] = 0x7fffffff;
    }
    float tv = -FTA_INF;
    int ti = 0x7fffffff;
    int cnt = 0;
    const float rl = row_lse[row];
    {
        // ranking key = value + log2(b / valid count), so its avg is 2^(key - rl) / b
        const float at = fta_exp2(tau_key[row] - rl) / (float)bsz;
        tv = at - fabsf(at) * 0x1p-8f;
    }
    float thr_norm = -FTA_INF, thr_log = -FTA_INF;
    auto set_thr = [&] __attribute__((always_inline)) () {
        const float t = tv * (float)bsz;
        thr_norm = t - fabsf(t) * 9.5367431640625e-07f;
        thr_log = (thr_norm > 0.f) ? fta_log2(thr_norm) - 2.44140625e-04f : -FTA_INF;
        // the owner's pre-filter in the value domain: value >= rl + thr_log, lowered
        // by a margin far above the rounding of the sum
        const float pv = rl + thr_log;
        s_pre[wave][lane] = active ? pv - (0x1p-12f + fabsf(pv) * 0x1p-20f) : FTA_INF;
        s_cnt[wave][lane] = 0;
    };
    set_thr();
    auto wave_sync = [] __attribute__((always_inline)) () {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    };
    auto flush = [&] __attribute__((always_inline)) () {
        wave_sync();
        cnt = min(s_cnt[wave][lane], CAP);
        fta_topk_flush<KB, CAP, 1>(lv, li, cnt, cand_v[wave], cand_i[wave], lane, active, rl, thr_log, thr_norm, M,
                                   bsz, pad_head, pad_tail, m_out, threshold, tv, ti);
        wave_sync();
        set_thr();
        wave_sync();
    };
    wave_sync();
    // NC chunks of 64 entries per step, the next two steps' chunks loading
    // meanwhile (one step ahead left the selector waiting on HBM latency); the
    // pre-filter reads, slot atomics and parking stores of a step's chunks are
    // issued together, so their LDS latencies overlap.
    constexpr int NC = 4;
    auto load_step = [&] __attribute__((always_inline)) (int c0, uint2 (&e)[NC]) {
        if (c0 >= total) return;
        // the step's 256 entries lie in one chunk; entries past the end (still
        // inside the chunk) are masked where they are used
        const int j = c0 / kStreamChunk;
        int id = (j == 0) ? (int)sw : tab[j];
        if ((unsigned)id >= (unsigned)pool_chunks) id = (int)sw;
        const uint2* ent = pool + (int64_t)id * kStreamChunk + (c0 - j * kStreamChunk);
#pragma unroll
        for (int i = 0; i < NC; ++i) e[i] = ent[i * 64 + lane];
    };
    constexpr int SZ = NC * 64;
    uint2 ea[NC], eb[NC], ec[NC];  // steps c0, c0 + SZ, c0 + 2 SZ
    load_step(0, ea);
    load_step(SZ, eb);
    for (int c0 = 0; c0 < total; c0 += SZ) {
        load_step(c0 + 2 * SZ, ec);
        int owner[NC], m[NC];
        float x[NC];
        bool pend[NC];
#pragma unroll
        for (int i = 0; i < NC; ++i) {
            owner[i] = (int)(ea[i].y >> 16) & 63;
            m[i] = (int)(ea[i].y & 0xffffu);
            x[i] = __builtin_bit_cast(float, ea[i].x);
            const bool em = ((m[i] == 0) & (pad_head > 0)) | ((m[i] == M - 1) & (pad_tail > 0));
            pend[i] = (c0 + i * 64 + lane < total) & (em | (x[i] >= s_pre[wave][owner[i]]));
        }
        // park the step's entries; while some find their owner's list full,
        // merge every list (flush) and park those again
        for (;;) {
            int pos[NC];
#pragma unroll
            for (int i = 0; i < NC; ++i) pos[i] = pend[i] ? atomicAdd(&s_cnt[wave][owner[i]], 1) : CAP;
            bool any = false;
#pragma unroll
            for (int i = 0; i < NC; ++i) {
                const bool ok = pend[i] & (pos[i] < CAP);
                if (ok) {
                    cand_v[wave][pos[i]][owner[i]] = x[i];
                    cand_i[wave][pos[i]][owner[i]] = m[i];
                }
                pend[i] = pend[i] & !ok;
                any |= pend[i];
            }
            if (__ballot(any) == 0ull) break;
            flush();
        }
#pragma unroll
        for (int i = 0; i < NC; ++i) {
            ea[i] = eb[i];
            eb[i] = ec[i];
        }
    }
    flush();
    const int nrows = min(64, N - n0);
    if (nrows <= 0) return;
    fta_topk_emit<KB, CAP>(lv, li, m_out, M, bsz, pad_head, pad_tail, threshold, out_idx, out_raw, out_avg,
                           (int64_t)bh * N + n0, nrows, lane, active, row, cand_v[wave]);
}

// Zeroes the stream pool's chunk counter and the fallback tile count (ctrs[0],
// ctrs[1]) before a scoring launch.
__global__ void fta_stream_reset_kernel(int* __restrict__ ctrs) {
    if (threadIdx.x < 2) ctrs[threadIdx.x] = 0;
}

// Fallback for the tiles whose candidate streams ran out of pool (listed by
// fta_topk_stream_kernel): each workgroup takes listed tiles in turn, scores
// the tile's 256 queries into its own [M][256] slot of per-block values (the
// scoring kernel's code with the stream filter replaced by the value store, so
// every value is the same fp32 number the stream carried) and selects their
// top-k from the slot with the selector of the per-block-value path.  The
// results equal the stream path's (both selectors are exact); only the time
// differs.
template <int DT, int D, int KB, int SB>
__global__ __launch_bounds__(256, 1) void fta_stream_fallback_kernel(ScoreArgs a, const int* __restrict__ ovf_list,
                                                                    const int* __restrict__ ovf_cnt,
                                                                    float* __restrict__ slots, int m_out,
                                                                    float threshold, int32_t* __restrict__ out_idx,
                                                                    float* __restrict__ out_raw,
                                                                    float* __restrict__ out_avg) {
    // the listed tiles (count and ids clamped to the grid of the scoring launch)
    const int n = min(__builtin_amdgcn_readfirstlane(*ovf_cnt), a.total);
    if ((int)blockIdx.x >= n) return;
    float* slot = slots + (int64_t)blockIdx.x * 256 * a.M;
    a.blk_lse = slot;
    a.blk_ld = 256;
    a.kgroups = 0;
    a.tau_idx = nullptr;
    for (int r = blockIdx.x; r < n; r += gridDim.x) {
        const int tile = __builtin_amdgcn_readfirstlane(ovf_list[r]);
        if ((unsigned)tile >= (unsigned)a.total) continue;  // workgroup-uniform
        fta_score_tile<DT, D, 0, 2, false, SB>(a, tile);
        __syncthreads();  // the slot is complete
        const int bh = tile / a.qtiles, qt = tile - bh * a.qtiles;
        const int64_t r0 = (int64_t)bh * a.N + qt * 256;
        const int rows = min(256, a.N - qt * 256);
        fta_topk_rows<KB, 1>(slot, 0, 0, a.row_lse + r0, 256, rows, a.M, m_out, a.bsz, a.pad_head, a.pad_tail,
                             threshold, out_idx + r0 * m_out, out_raw + r0 * m_out, out_avg + r0 * m_out, nullptr,
                             0);
        __syncthreads();  // the slot is free for the next tile
    }
}

// Slow general path for m_out > 64: one workgroup per row, bitonic sort of the
// M (<= 4096) 64-bit keys (orderable avg bits, ~index) in LDS.
__device__ __forceinline__ uint32_t fta_orderable(float f) {
    const uint32_t u = __builtin_bit_cast(uint32_t, f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float fta_unorderable(uint32_t u) {
    return __builtin_bit_cast(float, (u & 0x80000000u) ? (u & 0x7fffffffu) : ~u);
}

template <int MODE>
__global__ __launch_bounds__(256) void fta_topk_select_sort_kernel(
    const float* __restrict__ in, int64_t stride_row, int64_t stride_m, const float* __restrict__ row_lse,
    int N, int M, int m_out, int bsz, int pad_head, int pad_tail, float threshold,
    int32_t* __restrict__ out_idx, float* __restrict__ out_raw, float* __restrict__ out_avg) {
    __shared__ unsigned long long keys[4096];
    __shared__ int s_cut;
    const int row = blockIdx.x;
    int S = 1;
    while (S < M) S <<= 1;
    int64_t bh = row / N, n = row - (row / N) * N;
    for (int m = threadIdx.x; m < S; m += 256) {
        unsigned long long key = 0ull;
        if (m < M) {
            float raw;
            if (MODE == 0)
                raw = in[(int64_t)row * stride_row + m * stride_m];
            else
                raw = fta_exp2(in[(bh * M + m) * (int64_t)N + n] - row_lse[row]);
            const float avg = raw / (float)fta_valid_count(m, M, bsz, pad_head, pad_tail);
            key = ((unsigned long long)fta_orderable(avg) << 32) | (unsigned long long)(0xffffffffu - (uint32_t)m);
        }
        keys[m] = key;
    }
    __syncthreads();
    for (int size = 2; size <= S; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            for (int i = threadIdx.x; i < S; i += 256) {
                const int j = i ^ stride;
                if (j > i) {
                    const bool desc = (i & size) == 0;
                    const unsigned long long a = keys[i], bb = keys[j];
                    if (desc ? (a < bb) : (a > bb)) {
                        keys[i] = bb;
                        keys[j] = a;
                    }
                }
            }
            __syncthreads();
        }
    }
    if (threadIdx.x == 0) {
        float cs = 0.f;
        int cut = m_out;
        for (int p = 0; p < m_out; ++p) {
            const unsigned long long key = keys[p];
            const int id = (int)(0xffffffffu - (uint32_t)(key & 0xffffffffull));
            const float avg = fta_unorderable((uint32_t)(key >> 32));
            cs = __fadd_rn(cs, __fmul_rn(avg, (float)fta_valid_count(id, M, bsz, pad_head, pad_tail)));
            if (cs >= threshold) {
                cut = p + 1;
                break;
            }
        }
        s_cut = cut;
    }
    __syncthreads();
    const int cut = s_cut;
    for (int p = threadIdx.x; p < m_out; p += 256) {
        const unsigned long long key = keys[p];
        const int id = (int)(0xffffffffu - (uint32_t)(key & 0xffffffffull));
        const float avg = fta_unorderable((uint32_t)(key >> 32));
        const bool keep = p < cut;
        const int64_t o = (int64_t)row * m_out + p;
        out_idx[o] = keep ? id : -1;
        out_avg[o] = keep ? avg : 0.f;
        out_raw[o] = keep ? __fmul_rn(avg, (float)fta_valid_count(id, M, bsz, pad_head, pad_tail)) : 0.f;
    }
}

// ----------------------------------------------------------------------------
// Host launchers (extern "C" ABI, declared in include/fta.h)
// ----------------------------------------------------------------------------
#include "fta_host.h"

#include <cmath>

namespace {

// The pipelined scoring kernel serves b = 64 and b = 128 with D <= 128 (run as 64
// or 128 columns, the columns past D multiplied by zero q columns) and a K token
// stride whose 64-row offsets fit 32 bits.
bool score_pipe_ok(int bsz, int Dk, const int64_t* ks) {
    return (bsz == 64 || bsz == 128) && Dk <= 128 && ks[2] >= 0 && ks[2] <= (1 << 24);
}

// Candidate streams of the pipelined kernel (STREAM = true), laid out in the
// workspace by stream_layout: per-wave entry counts, chunk tables, the two
// counters (pool chunks taken, fallback tiles), the fallback tile list, row
// totals, tau keys, the fallback slots and the chunk pool (the rest of the
// workspace).  waves = B * H * ceil(N / 256) * 4.
struct StreamBufs {
    uint2* pool = nullptr;
    int* count = nullptr;
    int* tab = nullptr;
    int* ctrs = nullptr;
    int* ovf_list = nullptr;
    float* tau_key = nullptr;
    float* slots = nullptr;
    int m_out = 0;
    int maxch = 0;
    int pool_chunks = 0;
};

// Fallback slots ([M][256] fp32 each): the fallback kernel's workgroups.
constexpr int kStreamSlots = 64;

int64_t stream_waves(int B, int H, int N) { return (int64_t)B * H * ((N + 255) / 256) * 4; }

ScoreArgs score_args(const void* q, const void* k, int B, int H, int N, int D, const int64_t* qs, const int64_t* ks,
                     int M, int bsz, int pad_head, int pad_tail, float scale, float* blk_lse, float* row_lse,
                     int kgroups, int32_t* tau, const StreamBufs& sb) {
    ScoreArgs a;
    a.q = (const uint16_t*)q;
    a.k = (const uint16_t*)k;
    a.q_sb = qs[0];
    a.q_sh = qs[1];
    a.q_sn = qs[2];
    a.k_sb = ks[0];
    a.k_sh = ks[1];
    a.k_sn = ks[2];
    a.H = H;
    a.N = N;
    a.Dreal = D;
    a.M = M;
    a.bsz = bsz;
    a.pad_head = pad_head;
    a.pad_tail = pad_tail;
    a.c = scale * 1.4426950408889634f;
    a.blk_lse = blk_lse;
    a.blk_ld = 0;
    a.row_lse = row_lse;
    a.qtiles = (N + 255) / 256;
    a.total = a.qtiles * B * H;
    a.kgroups = kgroups;
    a.tau_idx = tau;
    a.pool = sb.pool;
    a.count = sb.count;
    a.tau_key = sb.tau_key;
    a.chunk_tab = sb.tab;
    a.pool_ctr = sb.ctrs;
    a.pool_chunks = sb.pool_chunks;
    a.maxch = sb.maxch;
    return a;
}

template <int DT>
int launch_score_lse_dt(const void* q, const void* k, int B, int H, int N, int D, int Dk, const int64_t* qs,
                        const int64_t* ks, int M, int bsz, int pad_head, int pad_tail, float scale,
                        float* blk_lse, float* row_lse, int kgroups, int32_t* tau, const StreamBufs& sb,
                        hipStream_t st) {
    const int qtiles = (N + 255) / 256;
    const int total = qtiles * B * H;
    const float c = scale * 1.4426950408889634f;
    const bool pipe = score_pipe_ok(bsz, Dk, ks);
    if (sb.pool != nullptr && !pipe) return fta::arg_error("block_score: candidate streams need the pipelined kernel");
    if (sb.pool != nullptr) {
        hipLaunchKernelGGL(fta_stream_reset_kernel, dim3(1), dim3(64), 0, st, sb.ctrs);
        int rc = fta::check_launch("fta_stream_reset_kernel");
        if (rc != FTA_OK) return rc;
    }
    const ScoreArgs sa = score_args(q, k, B, H, N, D, qs, ks, M, bsz, pad_head, pad_tail, scale, blk_lse, row_lse,
                                    kgroups, tau, sb);
#define FTA_LAUNCH_PIPE_SB(DK, NG, GT, GH, SB)                                                             \
    hipLaunchKernelGGL((fta_block_score_lse_pipe_kernel<DT, (DK <= 64) ? 64 : 128, NG, GT, GH, SB>),        \
                       dim3(total), dim3(256), 0, st, sa)
#define FTA_LAUNCH_PIPE(DK, NG, GT, GH)                                                                    \
    do {                                                                                                   \
        if (bsz == 64)                                                                                     \
            FTA_LAUNCH_PIPE_SB(DK, NG, GT, GH, 1);                                                         \
        else                                                                                               \
            FTA_LAUNCH_PIPE_SB(DK, NG, GT, GH, 2);                                                         \
    } while (0)
#define FTA_LAUNCH_SCORE(DK)                                                                               \
    if (pipe && sb.pool != nullptr && sb.m_out <= 8)                                                       \
        FTA_LAUNCH_PIPE(DK, 4, 2, false);                                                                  \
    else if (pipe && sb.pool != nullptr && sb.m_out <= 16)                                                 \
        FTA_LAUNCH_PIPE(DK, 4, 4, false);                                                                  \
    else if (pipe && sb.pool != nullptr)                                                                   \
        FTA_LAUNCH_PIPE(DK, 8, 4, true);                                                                   \
    else if (pipe)                                                                                         \
        FTA_LAUNCH_PIPE(DK, 0, 2, false);                                                                  \
    else if (bsz <= 64)                                                                                    \
        hipLaunchKernelGGL((fta_block_score_lse_fast_kernel<DT, DK, (DK > 128) ? 1 : 2>), dim3(total),    \
                           dim3(256 * (2 / ((DK > 128) ? 1 : 2))), 0, st,                                \
                           (const uint16_t*)q, (const uint16_t*)k, qs[0], qs[1], qs[2], ks[0], ks[1], ks[2], H, \
                           N, D, M, bsz, pad_head, pad_tail, c, blk_lse, row_lse, qtiles, total, kgroups, tau); \
    else                                                                                                   \
    hipLaunchKernelGGL((fta_block_score_lse_kernel<DT, DK>), dim3(total), dim3(256), 0, st,                \
                       (const uint16_t*)q, (const uint16_t*)k, qs[0], qs[1], qs[2], ks[0], ks[1], ks[2], H, N, \
                       D, M, bsz, pad_head, pad_tail, c, blk_lse, row_lse, qtiles, total, kgroups, tau)
    switch (Dk) {
        case 32: FTA_LAUNCH_SCORE(32); break;
        case 64: FTA_LAUNCH_SCORE(64); break;
        case 96: FTA_LAUNCH_SCORE(96); break;
        case 128: FTA_LAUNCH_SCORE(128); break;
        case 160: FTA_LAUNCH_SCORE(160); break;
        case 256: FTA_LAUNCH_SCORE(256); break;
        default: return fta::arg_error("block_score: unsupported head dim");
    }
#undef FTA_LAUNCH_SCORE
#undef FTA_LAUNCH_PIPE
#undef FTA_LAUNCH_PIPE_SB
    return fta::check_launch("fta_block_score_lse_kernel");
}

int launch_score_lse(const void* q, const void* k, int dtype, int B, int H, int N, int D, const int64_t* qs,
                     const int64_t* ks, int M, int bsz, int pad_head, int pad_tail, float scale, float* blk_lse,
                     float* row_lse, int kgroups, int32_t* tau, hipStream_t st, const StreamBufs& sb = StreamBufs()) {
    const int Dk = fta::kernel_head_dim(D);
    if (Dk < 0) return fta::arg_error("block_score: head dim must be <= 256");
    if (D % 8 != 0) return fta::arg_error("block_score: head dim must be a multiple of 8");
    if (dtype == FTA_DTYPE_BF16)
        return launch_score_lse_dt<FTA_DTYPE_BF16>(q, k, B, H, N, D, Dk, qs, ks, M, bsz, pad_head, pad_tail, scale,
                                                   blk_lse, row_lse, kgroups, tau, sb, st);
    if (dtype == FTA_DTYPE_F16)
        return launch_score_lse_dt<FTA_DTYPE_F16>(q, k, B, H, N, D, Dk, qs, ks, M, bsz, pad_head, pad_tail, scale,
                                                  blk_lse, row_lse, kgroups, tau, sb, st);
    return fta::arg_error("block_score: dtype must be bf16 or fp16");
}

template <int MODE>
int launch_topk(const float* in, int64_t stride_row, int64_t stride_m, const float* row_lse, int N, int rows,
                int M, int m_out, int bsz, int pad_head, int pad_tail, float threshold, int32_t* idx, float* raw,
                float* avg, const int32_t* tau, hipStream_t st) {
    if (rows == 0) return FTA_OK;
    if (m_out <= 64) {
        const int grid = (rows + 255) / 256;
#define FTA_LAUNCH_TOPK(KB)                                                                                \
    hipLaunchKernelGGL((fta_topk_select_kernel<KB, MODE>), dim3(grid), dim3(256), 0, st, in, stride_row,   \
                       stride_m, row_lse, N, rows, M, m_out, bsz, pad_head, pad_tail, threshold, idx, raw, avg, tau)
        if (m_out <= 8)
            FTA_LAUNCH_TOPK(8);
        else if (m_out <= 16)
            FTA_LAUNCH_TOPK(16);
        else if (m_out <= 32)
            FTA_LAUNCH_TOPK(32);
        else
            FTA_LAUNCH_TOPK(64);
#undef FTA_LAUNCH_TOPK
    } else {
        hipLaunchKernelGGL((fta_topk_select_sort_kernel<MODE>), dim3(rows), dim3(256), 0, st, in, stride_row,
                           stride_m, row_lse, N, M, m_out, bsz, pad_head, pad_tail, threshold, idx, raw, avg);
    }
    return fta::check_launch("fta_topk_select_kernel");
}

}  // namespace

extern "C" {

int fta_block_score_lse(const void* q, const void* k, int dtype, int B, int H, int N, int D,
                        const int64_t* q_strides, const int64_t* k_strides, int score_block_size, int pad_head,
                        int pad_tail, float scale, float* blk_lse, float* row_lse, void* stream) {
    FTA_TRY_BEGIN
    int M = 0;
    int st = fta::check_score_args(B, H, N, D, score_block_size, pad_head, pad_tail, &M);
    if (st != FTA_OK) return st;
    if (!q || !k || !blk_lse || !row_lse) return fta::arg_error("block_score_lse: null pointer");
    return launch_score_lse(q, k, dtype, B, H, N, D, q_strides, k_strides, M, score_block_size, pad_head, pad_tail,
                            scale, blk_lse, row_lse, 0, nullptr, (hipStream_t)stream);
    FTA_TRY_END
}

size_t fta_block_score_workspace_size(int B, int H, int N, int M) {
    return fta::align_up((size_t)B * H * M * N * sizeof(float)) + fta::align_up((size_t)B * H * N * sizeof(float));
}

int fta_block_score(const void* q, const void* k, int dtype, int B, int H, int N, int D, const int64_t* q_strides,
                    const int64_t* k_strides, int score_block_size, int pad_head, int pad_tail, float scale,
                    float* scores, void* workspace, size_t workspace_bytes, void* stream) {
    FTA_TRY_BEGIN
    int M = 0;
    int st = fta::check_score_args(B, H, N, D, score_block_size, pad_head, pad_tail, &M);
    if (st != FTA_OK) return st;
    if (!q || !k || !scores) return fta::arg_error("block_score: null pointer");
    if (workspace_bytes < fta_block_score_workspace_size(B, H, N, M))
        return fta::arg_error("block_score: workspace too small");
    float* blk_lse = (float*)workspace;
    float* row_lse = (float*)((char*)workspace + fta::align_up((size_t)B * H * M * N * sizeof(float)));
    hipStream_t s = (hipStream_t)stream;
    st = launch_score_lse(q, k, dtype, B, H, N, D, q_strides, k_strides, M, score_block_size, pad_head, pad_tail,
                          scale, blk_lse, row_lse, 0, nullptr, s);
    if (st != FTA_OK) return st;
    const int tn = (N + 63) / 64, tm = (M + 63) / 64;
    if ((int64_t)B * H * tn * tm > 0) {
        hipLaunchKernelGGL(fta_block_normalize_kernel, dim3(B * H * tn * tm), dim3(256), 0, s, blk_lse, row_lse,
                           scores, N, M, tn, tm);
    }
    return fta::check_launch("fta_block_normalize_kernel");
    FTA_TRY_END
}

int fta_topk_select(const float* block_scores, int64_t rows, int M, int64_t stride_row, int64_t stride_m,
                    int max_topk, int score_block_size, int pad_head, int pad_tail, float threshold,
                    int32_t* topk_indices, float* topk_raw, float* topk_avg, void* stream) {
    FTA_TRY_BEGIN
    if (M <= 0) return fta::arg_error("topk_select: M must be positive");
    if (M > 4096) return fta::unsupported("topk_select: M exceeds 4096");
    if (score_block_size <= 0) return fta::arg_error("topk_select: score_block_size must be positive");
    if (pad_head < 0 || pad_tail < 0 || pad_head >= score_block_size || pad_tail >= score_block_size)
        return fta::arg_error("topk_select: bad padding");
    if (max_topk < 0) return fta::arg_error("topk_select: max_topk must be >= 0");
    if (rows < 0 || rows > 0x7fffffff) return fta::arg_error("topk_select: bad row count");
    const int m_out = (max_topk > 0 && max_topk < M) ? max_topk : M;
    return launch_topk<0>(block_scores, stride_row, stride_m, nullptr, 1, (int)rows, M, m_out, score_block_size,
                          pad_head, pad_tail, threshold, topk_indices, topk_raw, topk_avg, nullptr, (hipStream_t)stream);
    FTA_TRY_END
}

}  // extern "C"

namespace {
// Candidate-stream workspace geometry (stream_layout): everything but the
// chunk pool has a fixed size; the pool takes the rest of the workspace.
struct StreamGeo {
    int64_t waves, tiles;
    int maxch;
    size_t fixed;
};
StreamGeo stream_geo(int B, int H, int N, int M) {
    StreamGeo g;
    g.waves = stream_waves(B, H, N);
    g.tiles = g.waves / 4;
    g.maxch = (64 * M + kStreamChunk - 1) / kStreamChunk + 1;  // a wave never needs more chunks
    const size_t rows = (size_t)B * H * N;
    g.fixed = fta::align_up(g.waves * sizeof(int)) + fta::align_up(g.waves * g.maxch * sizeof(int)) +
              fta::align_up(4 * sizeof(int)) + fta::align_up(g.tiles * sizeof(int)) +
              2 * fta::align_up(rows * sizeof(float)) +
              fta::align_up((size_t)kStreamSlots * 256 * M * sizeof(float));
    return g;
}
constexpr size_t kChunkBytes = (size_t)kStreamChunk * sizeof(uint2);
// The least workspace of the stream path: one chunk per wave.
size_t stream_min_bytes(int B, int H, int N, int M) {
    const StreamGeo g = stream_geo(B, H, N, M);
    return g.fixed + (size_t)g.waves * kChunkBytes;
}
// The recommended workspace of the stream path: a pool for the expected number
// of stream entries, E = m_out (1 + 2 ln(M / m_out)) per query (at most M; a
// block enters a query's stream when it may still be in its top m_out, which
// for blocks in random order happens about m_out ln(M / m_out) times beyond
// the first m_out; the filter's bound is looser than the exact m_out-th key,
// hence the factor 2), plus half a chunk per wave for partly filled chunks.
// Inputs that need more run their overflowing tiles through the fallback kernel.
size_t stream_rec_bytes(int B, int H, int N, int M, int m_out) {
    const StreamGeo g = stream_geo(B, H, N, M);
    double e = (m_out >= M) ? (double)M : (double)m_out * (1.0 + 2.0 * std::log((double)M / (double)m_out));
    if (e > (double)M) e = (double)M;
    const double entries = (double)B * H * N * std::ceil(e) + (double)g.waves * (kStreamChunk / 2);
    int64_t chunks = (int64_t)std::ceil(entries / kStreamChunk);
    if (chunks < g.waves) chunks = g.waves;
    if (chunks > g.waves * g.maxch) chunks = g.waves * g.maxch;
    return g.fixed + (size_t)chunks * kChunkBytes;
}
// The per-block value path: [BH][M][N] values + row totals + tau ids.
size_t full_bytes(int B, int H, int N, int M) {
    return fta_block_score_workspace_size(B, H, N, M) + fta::align_up((size_t)B * H * N * sizeof(int32_t));
}
}  // namespace

extern "C" {

size_t fta_topk_score_workspace_size(int B, int H, int N, int M) {
    if (B <= 0 || H <= 0 || N <= 0 || M <= 0) return 0;
    const size_t full = full_bytes(B, H, N, M);
    const size_t strm = stream_rec_bytes(B, H, N, M, M < kStreamMaxTopk ? M : kStreamMaxTopk);
    return full > strm ? full : strm;
}

size_t fta_topk_score_workspace_size_ex(int B, int H, int N, int D, int score_block_size, int pad_head,
                                        int pad_tail, int max_topk) {
    int M = 0;
    if (fta::check_score_args(B, H, N, D, score_block_size, pad_head, pad_tail, &M) != FTA_OK || max_topk < 0)
        return 0;
    const int m_out = (max_topk > 0 && max_topk < M) ? max_topk : M;
    const int64_t ks[3] = {0, 0, 0};  // a token stride within the pipelined kernel's range
    if (m_out <= kStreamMaxTopk && score_pipe_ok(score_block_size, fta::kernel_head_dim(D), ks))
        return stream_rec_bytes(B, H, N, M, m_out);
    return full_bytes(B, H, N, M);
}

size_t fta_topk_score_workspace_min(int B, int H, int N, int D, int score_block_size, int pad_head, int pad_tail,
                                    int max_topk) {
    int M = 0;
    if (fta::check_score_args(B, H, N, D, score_block_size, pad_head, pad_tail, &M) != FTA_OK || max_topk < 0)
        return 0;
    const int m_out = (max_topk > 0 && max_topk < M) ? max_topk : M;
    const int64_t ks[3] = {0, 0, 0};
    if (m_out <= kStreamMaxTopk && score_pipe_ok(score_block_size, fta::kernel_head_dim(D), ks))
        return stream_min_bytes(B, H, N, M);
    return full_bytes(B, H, N, M);
}

}  // extern "C"

namespace {
// fta_topk_score's workspace as candidate streams (StreamBufs), in this order:
// per-wave counts, chunk tables, counters, fallback tile list, row totals, tau
// keys, fallback slots, chunk pool (the rest of the workspace).
StreamBufs stream_layout(void* workspace, size_t workspace_bytes, int B, int H, int N, int M, int m_out,
                         float** row_lse) {
    const StreamGeo g = stream_geo(B, H, N, M);
    const size_t rows = (size_t)B * H * N;
    char* p = (char*)workspace;
    StreamBufs sb;
    sb.count = (int*)p;
    p += fta::align_up(g.waves * sizeof(int));
    sb.tab = (int*)p;
    p += fta::align_up(g.waves * g.maxch * sizeof(int));
    sb.ctrs = (int*)p;
    p += fta::align_up(4 * sizeof(int));
    sb.ovf_list = (int*)p;
    p += fta::align_up(g.tiles * sizeof(int));
    *row_lse = (float*)p;
    p += fta::align_up(rows * sizeof(float));
    sb.tau_key = (float*)p;
    p += fta::align_up(rows * sizeof(float));
    sb.slots = (float*)p;
    p += fta::align_up((size_t)kStreamSlots * 256 * M * sizeof(float));
    sb.pool = (uint2*)p;
    const size_t pool_bytes = workspace_bytes - (size_t)(p - (char*)workspace);
    const int64_t chunks = (int64_t)(pool_bytes / kChunkBytes);
    sb.pool_chunks = (int)(chunks < (int64_t)0x7fffffff ? chunks : (int64_t)0x7fffffff);
    sb.maxch = g.maxch;
    sb.m_out = m_out;
    return sb;
}

// The selector over the candidate streams (fta_topk_stream_kernel), then the
// fallback kernel for tiles whose streams ran out of pool (it returns at once
// when there are none).
template <int DT>
int launch_stream_select_dt(const ScoreArgs& sa, int Dk, const StreamBufs& sb, int m_out, float threshold,
                            int32_t* idx, float* raw, float* avg, hipStream_t s) {
    const int qtiles = sa.qtiles;
#define FTA_LAUNCH_STREAM(KB)                                                                                     \
    hipLaunchKernelGGL(fta_topk_stream_kernel<KB>, dim3((unsigned)sa.total), dim3(256), 0, s, sb.pool, sb.count, \
                       sb.tab, sb.maxch, sb.tau_key, sa.row_lse, sa.N, qtiles, sa.M, m_out, sa.bsz, sa.pad_head,  \
                       sa.pad_tail, threshold, idx, raw, avg, sb.ovf_list, sb.ctrs + 1, sb.pool_chunks)
    if (m_out <= 8)
        FTA_LAUNCH_STREAM(8);
    else if (m_out <= 16)
        FTA_LAUNCH_STREAM(16);
    else
        FTA_LAUNCH_STREAM(32);
#undef FTA_LAUNCH_STREAM
    int rc = fta::check_launch("fta_topk_stream_kernel");
    if (rc != FTA_OK) return rc;
    const int grid = sa.total < kStreamSlots ? sa.total : kStreamSlots;
#define FTA_LAUNCH_FALLBACK(DK, SB)                                                                             \
    hipLaunchKernelGGL((fta_stream_fallback_kernel<DT, DK, 32, SB>), dim3(grid), dim3(256), 0, s, sa, sb.ovf_list, \
                       sb.ctrs + 1, sb.slots, m_out, threshold, idx, raw, avg)
    if (Dk <= 64 && sa.bsz == 64)
        FTA_LAUNCH_FALLBACK(64, 1);
    else if (Dk <= 64)
        FTA_LAUNCH_FALLBACK(64, 2);
    else if (sa.bsz == 64)
        FTA_LAUNCH_FALLBACK(128, 1);
    else
        FTA_LAUNCH_FALLBACK(128, 2);
#undef FTA_LAUNCH_FALLBACK
    return fta::check_launch("fta_stream_fallback_kernel");
}

// Shared checks of the fta_topk_score entry points; sets M, m_out and whether
// the candidate-stream path applies, and checks the workspace for that path.
int topk_score_checks(int B, int H, int N, int D, int bsz, int pad_head, int pad_tail, int max_topk,
                      const int64_t* k_strides, size_t workspace_bytes, int* M, int* m_out, bool* streams) {
    int st = fta::check_score_args(B, H, N, D, bsz, pad_head, pad_tail, M);
    if (st != FTA_OK) return st;
    if (*M > 4096) return fta::unsupported("topk_score: M exceeds 4096");
    if (max_topk < 0) return fta::arg_error("topk_score: max_topk must be >= 0");
    *m_out = (max_topk > 0 && max_topk < *M) ? max_topk : *M;
    *streams = *m_out <= kStreamMaxTopk && score_pipe_ok(bsz, fta::kernel_head_dim(D), k_strides);
    const size_t need = *streams ? stream_min_bytes(B, H, N, *M) : full_bytes(B, H, N, *M);
    if (workspace_bytes < need)
        return fta::arg_error("topk_score: workspace too small (see fta_topk_score_workspace_size_ex)");
    return FTA_OK;
}

int stream_select(const void* q, const void* k, int dtype, int B, int H, int N, int D, const int64_t* qs,
                  const int64_t* ks, int bsz, int pad_head, int pad_tail, float scale, int M, int m_out,
                  float threshold, int32_t* idx, float* raw, float* avg, void* workspace, size_t workspace_bytes,
                  hipStream_t s) {
    float* row_lse = nullptr;
    const StreamBufs sb = stream_layout(workspace, workspace_bytes, B, H, N, M, m_out, &row_lse);
    const ScoreArgs sa =
        score_args(q, k, B, H, N, D, qs, ks, M, bsz, pad_head, pad_tail, scale, nullptr, row_lse, 0, nullptr, sb);
    const int Dk = fta::kernel_head_dim(D);
    if (dtype == FTA_DTYPE_BF16)
        return launch_stream_select_dt<FTA_DTYPE_BF16>(sa, Dk, sb, m_out, threshold, idx, raw, avg, s);
    if (dtype == FTA_DTYPE_F16)
        return launch_stream_select_dt<FTA_DTYPE_F16>(sa, Dk, sb, m_out, threshold, idx, raw, avg, s);
    return fta::arg_error("topk_score: dtype must be bf16 or fp16");
}
}  // namespace

extern "C" {

int fta_topk_score_candidates(const void* q, const void* k, int dtype, int B, int H, int N, int D,
                              const int64_t* q_strides, const int64_t* k_strides, int score_block_size, int pad_head,
                              int pad_tail, float scale, int max_topk, void* workspace, size_t workspace_bytes,
                              void* stream) {
    FTA_TRY_BEGIN
    int M = 0, m_out = 0;
    bool streams = false;
    int st = topk_score_checks(B, H, N, D, score_block_size, pad_head, pad_tail, max_topk, k_strides,
                               workspace_bytes, &M, &m_out, &streams);
    if (st != FTA_OK) return st;
    if (!streams)
        return fta::unsupported("topk_score_candidates: needs b = 64 or 128, D <= 128 and at most 32 blocks per query");
    float* row_lse = nullptr;
    const StreamBufs sb = stream_layout(workspace, workspace_bytes, B, H, N, M, m_out, &row_lse);
    return launch_score_lse(q, k, dtype, B, H, N, D, q_strides, k_strides, M, score_block_size, pad_head, pad_tail,
                            scale, nullptr, row_lse, 0, nullptr, (hipStream_t)stream, sb);
    FTA_TRY_END
}

int fta_topk_select_candidates(const void* q, const void* k, int dtype, int B, int H, int N, int D,
                               const int64_t* q_strides, const int64_t* k_strides, int score_block_size,
                               int pad_head, int pad_tail, float scale, int max_topk, float threshold,
                               int32_t* topk_indices, float* topk_raw, float* topk_avg, void* workspace,
                               size_t workspace_bytes, void* stream) {
    FTA_TRY_BEGIN
    int M = 0, m_out = 0;
    bool streams = false;
    int st = topk_score_checks(B, H, N, D, score_block_size, pad_head, pad_tail, max_topk, k_strides,
                               workspace_bytes, &M, &m_out, &streams);
    if (st != FTA_OK) return st;
    if (!streams)
        return fta::unsupported("topk_select_candidates: needs b = 64 or 128, D <= 128 and at most 32 blocks per query");
    if (!topk_indices || !topk_raw || !topk_avg) return fta::arg_error("topk_select_candidates: null pointer");
    return stream_select(q, k, dtype, B, H, N, D, q_strides, k_strides, score_block_size, pad_head, pad_tail, scale,
                         M, m_out, threshold, topk_indices, topk_raw, topk_avg, workspace, workspace_bytes,
                         (hipStream_t)stream);
    FTA_TRY_END
}

int fta_topk_score(const void* q, const void* k, int dtype, int B, int H, int N, int D, const int64_t* q_strides,
                   const int64_t* k_strides, int score_block_size, int pad_head, int pad_tail, float scale,
                   int max_topk, float threshold, int32_t* topk_indices, float* topk_raw, float* topk_avg,
                   void* workspace, size_t workspace_bytes, void* stream) {
    FTA_TRY_BEGIN
    int M = 0, m_out = 0;
    bool streams = false;
    int st = topk_score_checks(B, H, N, D, score_block_size, pad_head, pad_tail, max_topk, k_strides,
                               workspace_bytes, &M, &m_out, &streams);
    if (st != FTA_OK) return st;
    hipStream_t s = (hipStream_t)stream;
    if (streams) {
        // candidate streams: no [BH][M][N] intermediate
        float* row_lse = nullptr;
        const StreamBufs sb = stream_layout(workspace, workspace_bytes, B, H, N, M, m_out, &row_lse);
        st = launch_score_lse(q, k, dtype, B, H, N, D, q_strides, k_strides, M, score_block_size, pad_head, pad_tail,
                              scale, nullptr, row_lse, 0, nullptr, s, sb);
        if (st != FTA_OK) return st;
        return stream_select(q, k, dtype, B, H, N, D, q_strides, k_strides, score_block_size, pad_head, pad_tail,
                             scale, M, m_out, threshold, topk_indices, topk_raw, topk_avg, workspace, workspace_bytes,
                             s);
    }
    float* blk_lse = (float*)workspace;
    float* row_lse = (float*)((char*)workspace + fta::align_up((size_t)B * H * M * N * sizeof(float)));
    int32_t* tau = (int32_t*)((char*)workspace + fta_block_score_workspace_size(B, H, N, M));
    const int kgroups = (m_out <= 64) ? m_out : 0;
    st = launch_score_lse(q, k, dtype, B, H, N, D, q_strides, k_strides, M, score_block_size, pad_head, pad_tail,
                          scale, blk_lse, row_lse, kgroups, tau, s);
    if (st != FTA_OK) return st;
    return launch_topk<1>(blk_lse, 0, 0, row_lse, N, B * H * N, M, m_out, score_block_size, pad_head, pad_tail,
                          threshold, topk_indices, topk_raw, topk_avg, kgroups ? tau : nullptr, s);
    FTA_TRY_END
}

}  // extern "C"
