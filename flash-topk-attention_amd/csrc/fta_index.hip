// Index kernels: q-block merge, reverse index, count sorts and delta.
//
// All of them are deterministic: sums run in a fixed order and no result
// depends on atomic ordering (the reference's merge and reverse-index kernels,
// flash_topk_attn_v2/csrc/qblock_merge_kernel.cu:44-52 and
// csrc/build_reverse_indices_kernel.cu:19-25, are not).
#include "fta_common.h"
#include "fta_host.h"

// 256-thread exclusive scan; returns the exclusive prefix and writes the total.
__device__ __forceinline__ int fta_block_scan256(int v, int* s_tmp, int* total) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    int x = v;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const int y = __shfl_up(x, off, 64);
        if (lane >= off) x += y;
    }
    if (lane == 63) s_tmp[wave] = x;
    __syncthreads();
    int wbase = 0, tot = 0;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        const int t = s_tmp[w];
        if (w < wave) wbase += t;
        tot += t;
    }
    __syncthreads();
    *total = tot;
    return wbase + x - v;
}

// ----------------------------------------------------------------------------
// q-block merge (reference: flash_topk_attn_v2/qblock_merge.py:27-155,
// csrc/qblock_merge_kernel.cu:8-89).  One workgroup per (b, h, q-block) slice:
//   acc[id] += score over the slice's g*K (id, score) pairs in (row, slot) order,
//   positive entries sorted by (score desc, id asc), first W kept.
// ----------------------------------------------------------------------------
constexpr int kMergeChunk = 1024;  // staged (id, score) entries per step
constexpr int kUnionMax = 8192;    // largest union row (ids held in LDS: 32 KB)

__global__ __launch_bounds__(256) void fta_qblock_merge_kernel(const int32_t* __restrict__ idx,
                                                               const float* __restrict__ scr, int g, int K,
                                                               int Mt_arg, const int32_t* __restrict__ max_id,
                                                               int W, int32_t* __restrict__ out_idx,
                                                               float* __restrict__ out_scr,
                                                               int32_t* __restrict__ counts) {
    // block count: the argument, or (max id + 1) read from device memory, kept
    // within the 4096-entry histogram (a larger max is an error the host reports)
    const int Mt = max_id ? min(max(*max_id + 1, 1), 4096) : Mt_arg;
    __shared__ float acc[4096];
    __shared__ unsigned long long keys[4096];
    __shared__ int s_tmp[8];
    __shared__ int s_id[kMergeChunk];
    __shared__ float s_sc[kMergeChunk];
    // volatile: the owner test must re-read LDS after the atomic, and each
    // round must see the previous round's sums.
    volatile int* owner = reinterpret_cast<volatile int*>(keys);  // reused before the sort
    volatile float* vacc = acc;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t slice = blockIdx.x;
    const int32_t* ip = idx + slice * (int64_t)g * K;
    const float* sp = scr + slice * (int64_t)g * K;

    for (int m = tid; m < Mt; m += 256) acc[m] = 0.f;
    __syncthreads();

    // Entries are consumed in position order (row-major (row, slot)), which
    // keeps every id's fp32 sum in (row, slot) order.  All threads stage a
    // chunk of entries in LDS; wave 0 then adds 64 consecutive entries per
    // step (duplicates within a step are serialised in lane = position order).
    const int total = g * K;
    for (int e0 = 0; e0 < total; e0 += kMergeChunk) {
        const int n = min(kMergeChunk, total - e0);
        for (int e = tid; e < n; e += 256) {
            s_id[e] = ip[e0 + e];
            s_sc[e] = sp[e0 + e];
        }
        __syncthreads();
        if (wave == 0) {
            for (int j0 = 0; j0 < n; j0 += 64) {
                const int j = j0 + lane;
                const int id = (j < n) ? s_id[j] : -1;
                const float sc = (j < n) ? s_sc[j] : 0.f;
                // rounds: in each, the lowest remaining lane of every id adds its
                // entry, so an id's entries are added in lane (= position) order
                bool pending = id >= 0 && id < Mt;
                while (__ballot(pending) != 0ull) {
                    if (pending) owner[id] = 64;
                    if (pending) atomicMin(const_cast<int*>(&owner[id]), lane);
                    if (pending && owner[id] == lane) {
                        vacc[id] = __fadd_rn(vacc[id], sc);
                        pending = false;
                    }
                }
            }
        }
        __syncthreads();
    }

    // compact positive entries in id order
    int P = 0;
    for (int base = 0; base < Mt; base += 256) {
        const int m = base + tid;
        const float a = (m < Mt) ? acc[m] : 0.f;
        const int pos = (a > 0.f) ? 1 : 0;
        int tot;
        const int off = fta_block_scan256(pos, s_tmp, &tot);
        if (pos) {
            keys[P + off] = ((unsigned long long)__builtin_bit_cast(uint32_t, a) << 32) |
                            (unsigned long long)(0xffffffffu - (uint32_t)m);
        }
        P += tot;
    }
    int S = 1;
    while (S < P) S <<= 1;
    for (int i = P + tid; i < S; i += 256) keys[i] = 0ull;
    __syncthreads();
    for (int size = 2; size <= S; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            for (int i = tid; i < S; i += 256) {
                const int j = i ^ stride;
                if (j > i) {
                    const bool desc = (i & size) == 0;
                    const unsigned long long a = keys[i], b = keys[j];
                    if (desc ? (a < b) : (a > b)) {
                        keys[i] = b;
                        keys[j] = a;
                    }
                }
            }
            __syncthreads();
        }
    }
    const int keep = P < W ? P : W;
    int32_t* oi = out_idx + slice * (int64_t)W;
    float* os = out_scr ? out_scr + slice * (int64_t)W : nullptr;
    for (int p = tid; p < W; p += 256) {
        if (p < keep) {
            const unsigned long long key = keys[p];
            oi[p] = (int)(0xffffffffu - (uint32_t)(key & 0xffffffffull));
            if (os) os[p] = __builtin_bit_cast(float, (uint32_t)(key >> 32));
        } else {
            oi[p] = -1;
            if (os) os[p] = 0.f;
        }
    }
    if (counts && tid == 0) counts[slice] = keep;
}

// ----------------------------------------------------------------------------
// q-block merge, one wave per slice (used when g*K <= 4096).  Same results as
// fta_qblock_merge_kernel without an M-sized histogram:
//   1. the slice's valid entries (0 <= id < block count) are compacted and
//      sorted ascending by (id << 16 | position) in LDS (bitonic), so each
//      id's entries form one run in position order;
//   2. the first lane of a run sums it sequentially in that order (the same
//      fp32 additions, in the same order, as the histogram kernel);
//   3. positive sums are compacted and sorted by (score desc, id asc).
// No workgroup barrier: up to four waves, each on its own slice and LDS region.
// ----------------------------------------------------------------------------
constexpr int kMergeWaveMax = 4096;  // largest g*K of the one-wave path
// valid entries from which the one-wave path sums per id in an LDS histogram
// instead of sorting the entries (dense lists: few duplicate ids per 64)
constexpr int kMergeWaveHistNV = 384;

__device__ __forceinline__ void fta_wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Bitonic sort of arr[0, n) (n a power of two <= 64 * E) held in registers: lane
// l holds elements l*E .. l*E+E-1 (past n: `pad`, which sorts last).  Strides
// below E swap within a lane, larger ones exchange with lane l ^ (stride / E).
// Ascending, or descending with DESC.  The result is written back to arr.
template <typename K>
__device__ __forceinline__ K fta_shfl_xor_k(K v, int d) {
    if constexpr (sizeof(K) == 8) {
        const uint32_t lo = (uint32_t)v, hi = (uint32_t)(v >> 32);
        return ((K)(uint32_t)__shfl_xor((int)hi, d, 64) << 32) | (K)(uint32_t)__shfl_xor((int)lo, d, 64);
    } else {
        return (K)__shfl_xor((int)v, d, 64);
    }
}

template <int E, typename K, bool DESC>
__device__ __forceinline__ void fta_wave_sort_regs(K* arr, int n, K pad, int lane) {
    constexpr int NN = 64 * E;
    K v[E];
#pragma unroll
    for (int r = 0; r < E; ++r) {
        const int i = lane * E + r;
        v[r] = (i < n) ? arr[i] : pad;
    }
#pragma unroll
    for (int k = 2; k <= NN; k <<= 1) {
#pragma unroll
        for (int j = k >> 1; j > 0; j >>= 1) {
            if (j < E) {
#pragma unroll
                for (int r = 0; r < E; ++r) {
                    if ((r & j) == 0) {
                        const bool up = (((lane * E + r) & k) == 0) != DESC;
                        const K a = v[r], b = v[r | j];
                        const bool sw = up ? (a > b) : (a < b);
                        v[r] = sw ? b : a;
                        v[r | j] = sw ? a : b;
                    }
                }
            } else {
                const int d = j / E;
                const bool lower = (lane & d) == 0;
#pragma unroll
                for (int r = 0; r < E; ++r) {
                    const K p = fta_shfl_xor_k(v[r], d);
                    const bool up = (((lane * E + r) & k) == 0) != DESC;
                    v[r] = (lower == up) ? (v[r] < p ? v[r] : p) : (v[r] > p ? v[r] : p);
                }
            }
        }
    }
#pragma unroll
    for (int r = 0; r < E; ++r) {
        const int i = lane * E + r;
        if (i < n) arr[i] = v[r];
    }
}

// Sort arr[0, n) (n a power of two) across one wave: in registers up to 512
// elements, else bitonic in LDS.
template <typename K, bool DESC>
__device__ __forceinline__ void fta_wave_sort(K* arr, int n, K pad, int lane) {
    if (n <= 64) {
        fta_wave_sort_regs<1, K, DESC>(arr, n, pad, lane);
    } else if (n <= 128) {
        fta_wave_sort_regs<2, K, DESC>(arr, n, pad, lane);
    } else if (n <= 256) {
        fta_wave_sort_regs<4, K, DESC>(arr, n, pad, lane);
    } else if (n <= 512) {
        fta_wave_sort_regs<8, K, DESC>(arr, n, pad, lane);
    } else {
        for (int k = 2; k <= n; k <<= 1) {
            for (int j = k >> 1; j > 0; j >>= 1) {
                for (int t = lane; t < (n >> 1); t += 64) {
                    const int i = ((t & ~(j - 1)) << 1) | (t & (j - 1));
                    const K a = arr[i], b = arr[i + j];
                    if ((DESC ? (a < b) : (a > b)) == ((i & k) == 0)) {
                        arr[i] = b;
                        arr[i + j] = a;
                    }
                }
                fta_wave_sync();
            }
        }
    }
    fta_wave_sync();
}

__global__ __launch_bounds__(256) void fta_qblock_merge_wave_kernel(
    const int32_t* __restrict__ idx, const float* __restrict__ scr, int64_t num_slices, int g, int K, int NP,
    int Mt_arg, const int32_t* __restrict__ max_id, int W, int32_t* __restrict__ out_idx,
    float* __restrict__ out_scr, int32_t* __restrict__ counts) {
    extern __shared__ __align__(16) unsigned char smem[];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, wpb = blockDim.x >> 6;
    const int64_t slice = (int64_t)blockIdx.x * wpb + wave;
    if (slice >= num_slices) return;
    const int Mt = max_id ? min(max(*max_id + 1, 1), 4096) : Mt_arg;
    unsigned char* base = smem + (size_t)wave * NP * 16;
    unsigned long long* out = reinterpret_cast<unsigned long long*>(base);  // [NP]
    uint32_t* key = reinterpret_cast<uint32_t*>(base + (size_t)NP * 8);      // [NP]
    float* sc = reinterpret_cast<float*>(base + (size_t)NP * 12);            // [NP], by position
    const int n = g * K;
    const int32_t* ip = idx + slice * (int64_t)n;
    const float* sp = scr + slice * (int64_t)n;
    // valid entries are compacted (ballot) so that only next_pow2(#valid) keys are sorted
    int NV = 0;
    for (int r0 = 0; r0 < n; r0 += 64) {
        const int i = r0 + lane;
        bool valid = false;
        uint32_t kv = 0xffffffffu;
        if (i < n) {
            const int id = ip[i];
            sc[i] = sp[i];
            valid = id >= 0 && id < Mt;
            kv = ((uint32_t)id << 16) | (uint32_t)i;
        }
        const unsigned long long vm = __ballot(valid);
        if (valid) key[NV + __popcll(vm & ((1ull << lane) - 1ull))] = kv;
        NV += __popcll(vm);
    }
    int P = 0;
    if (NV >= kMergeWaveHistNV && Mt <= NP) {
        // Nearly every entry valid: per-id sums in an LDS histogram over the
        // Mt ids (in the `out` bytes) instead of a sort of NV keys.  Entries
        // are added in position order (compacted order; within 64, lowest lane
        // first through owner rounds), the same fp32 additions as the sorted
        // runs below.  The positive sums then go to the key / score bytes.
        volatile float* acc = reinterpret_cast<volatile float*>(base);              // [Mt]
        volatile int* owner = reinterpret_cast<volatile int*>(base + (size_t)NP * 4);  // [Mt]
        for (int m = lane; m < Mt; m += 64) acc[m] = 0.f;
        fta_wave_sync();
        for (int r0 = 0; r0 < NV; r0 += 64) {
            const int i = r0 + lane;
            bool pending = i < NV;
            const uint32_t kv = pending ? key[i] : 0u;
            const int id = (int)(kv >> 16);
            const float v = pending ? sc[kv & 0xffffu] : 0.f;
            while (__ballot(pending) != 0ull) {
                if (pending) owner[id] = 64;
                if (pending) atomicMin(const_cast<int*>(&owner[id]), lane);
                if (pending && owner[id] == lane) {
                    acc[id] = __fadd_rn(acc[id], v);
                    pending = false;
                }
            }
        }
        fta_wave_sync();
        out = reinterpret_cast<unsigned long long*>(base + (size_t)NP * 8);  // over key / sc
        for (int m0 = 0; m0 < Mt; m0 += 64) {
            const int m = m0 + lane;
            const float sum = (m < Mt) ? acc[m] : 0.f;
            const bool pos = sum > 0.f;
            const unsigned long long mask = __ballot(pos);
            if (pos)
                out[P + __popcll(mask & ((1ull << lane) - 1ull))] =
                    ((unsigned long long)__builtin_bit_cast(uint32_t, sum) << 32) |
                    (unsigned long long)(0xffffffffu - (uint32_t)m);
            P += __popcll(mask);
        }
    } else {
        int NS = 1;
        while (NS < NV) NS <<= 1;
        for (int i = NV + lane; i < NS; i += 64) key[i] = 0xffffffffu;
        fta_wave_sync();
        fta_wave_sort<uint32_t, false>(key, NS, 0xffffffffu, lane);
        for (int r0 = 0; r0 < NV; r0 += 64) {
            const int i = r0 + lane;
            const uint32_t kv = (i < NV) ? key[i] : 0xffffffffu;
            const uint32_t id = kv >> 16;
            const bool head = kv != 0xffffffffu && (i == 0 || (key[i - 1] >> 16) != id);
            float sum = 0.f;
            if (head)
                for (int j = i; j < NV && (key[j] >> 16) == id; ++j) sum = __fadd_rn(sum, sc[key[j] & 0xffffu]);
            const bool pos = head && sum > 0.f;
            const unsigned long long mask = __ballot(pos);
            const int off = __popcll(mask & ((1ull << lane) - 1ull));
            if (pos)
                out[P + off] = ((unsigned long long)__builtin_bit_cast(uint32_t, sum) << 32) |
                               (unsigned long long)(0xffffffffu - id);
            P += __popcll(mask);
        }
    }
    int S = 1;
    while (S < P) S <<= 1;
    for (int i = P + lane; i < S; i += 64) out[i] = 0ull;
    fta_wave_sync();
    fta_wave_sort<unsigned long long, true>(out, S, 0ull, lane);  // descending
    const int keep = P < W ? P : W;
    int32_t* oi = out_idx + slice * (int64_t)W;
    float* os = out_scr ? out_scr + slice * (int64_t)W : nullptr;
    for (int p = lane; p < W; p += 64) {
        if (p < keep) {
            const unsigned long long kv = out[p];
            oi[p] = (int)(0xffffffffu - (uint32_t)(kv & 0xffffffffull));
            if (os) os[p] = __builtin_bit_cast(float, (uint32_t)(kv >> 32));
        } else {
            oi[p] = -1;
            if (os) os[p] = 0.f;
        }
    }
    if (counts && lane == 0) counts[slice] = keep;
}

// ----------------------------------------------------------------------------
// q-block merge, one lane per slice, for g*K <= NMAX (32) entries (g = 1 or 2
// q-blocks of a few queries).  Same results as the kernels above: the lane
// adds each valid id's scores in position order (an entry joins the first
// earlier entry with its id), then insertion-sorts the positive sums by
// (score desc, id asc) in registers.  Replaces a 64-lane wave per slice, whose
// bitonic networks ran at 64 elements for these 16- or 32-entry slices.
// ----------------------------------------------------------------------------
template <int NMAX>
__global__ __launch_bounds__(256) void fta_qblock_merge_lane_kernel(
    const int32_t* __restrict__ idx, const float* __restrict__ scr, int64_t num_slices, int n, int Mt_arg,
    const int32_t* __restrict__ max_id, int W, int32_t* __restrict__ out_idx, float* __restrict__ out_scr,
    int32_t* __restrict__ counts) {
    // The workgroup's 256 slices are contiguous in HBM (n entries each): they are
    // read and their results written as whole blocks through LDS (rows padded to
    // NMAX + 1 words against bank conflicts), so every global access is
    // coalesced; one lane then works on one row.
    constexpr int RS = NMAX + 1;
    __shared__ int s_id[256 * RS];
    __shared__ float s_sc[256 * RS];
    __shared__ int s_keep[256];
    const int tid = threadIdx.x;
    const int64_t s0 = (int64_t)blockIdx.x * 256;
    const int ns = (int)min((int64_t)256, num_slices - s0);
    const int Mt = max_id ? min(max(*max_id + 1, 1), 4096) : Mt_arg;
    {
        const int32_t* ib = idx + s0 * n;
        const float* sb = scr + s0 * n;
        for (int e = tid; e < ns * n; e += 256) {
            const int r = e / n, c = e - r * n;
            s_id[r * RS + c] = ib[e];
            s_sc[r * RS + c] = sb[e];
        }
    }
    __syncthreads();
    int oid[NMAX];
    float osc[NMAX];
    int P = 0;
    if (tid < ns) {
        int id[NMAX];
        float sum[NMAX];
        int U = 0;  // distinct valid ids so far, in first-appearance order
#pragma unroll
        for (int j = 0; j < NMAX; ++j) {
            if (j < n) {
                const int m = s_id[tid * RS + j];
                const float sc = s_sc[tid * RS + j];
                if (m >= 0 && m < Mt) {
                    bool found = false;
#pragma unroll
                    for (int u = 0; u < NMAX; ++u)
                        if (u < U && id[u] == m && !found) {
                            sum[u] = __fadd_rn(sum[u], sc);
                            found = true;
                        }
                    if (!found) {
#pragma unroll
                        for (int u = 0; u < NMAX; ++u)
                            if (u == U) {
                                id[u] = m;
                                sum[u] = sc;
                            }
                        ++U;
                    }
                }
            }
        }
        // insertion sort of the positive sums: score desc, then id asc
#pragma unroll
        for (int u = 0; u < NMAX; ++u) {
            if (u < U && sum[u] > 0.f) {
                const float v = sum[u];
                const int m = id[u];
                // position = entries ranking above (v, m); shift the rest down one slot
                int pos = 0;
#pragma unroll
                for (int p = 0; p < NMAX; ++p)
                    if (p < P && (osc[p] > v || (osc[p] == v && oid[p] < m))) ++pos;
#pragma unroll
                for (int p = NMAX - 1; p > 0; --p)
                    if (p > pos && p <= P) {
                        osc[p] = osc[p - 1];
                        oid[p] = oid[p - 1];
                    }
#pragma unroll
                for (int p = 0; p < NMAX; ++p)
                    if (p == pos) {
                        osc[p] = v;
                        oid[p] = m;
                    }
                ++P;
            }
        }
    }
    __syncthreads();  // every lane has read its row
    const int keep = P < W ? P : W;
    if (tid < ns) {
#pragma unroll
        for (int p = 0; p < NMAX; ++p) {
            s_id[tid * RS + p] = oid[p];
            s_sc[tid * RS + p] = osc[p];
        }
        s_keep[tid] = keep;
        if (counts) counts[s0 + tid] = keep;
    }
    __syncthreads();
    // the block of ns x W outputs, -1 / 0 after each row's kept entries
    int32_t* ob = out_idx + s0 * W;
    float* sb = out_scr ? out_scr + s0 * W : nullptr;
    for (int e = tid; e < ns * W; e += 256) {
        const int r = e / W, c = e - r * W;
        const bool k = c < s_keep[r];  // then c < NMAX: inside the row
        const int a = r * RS + (k ? c : 0);
        ob[e] = k ? s_id[a] : -1;
        if (sb) sb[e] = k ? s_sc[a] : 0.f;
    }
}

// ----------------------------------------------------------------------------
// q-block merge, one wave per slice, for g*K > 512 entries over at most
// kMergeHistM blocks.  Same results as the kernels above: the wave adds its
// slice's entries 64 at a time into an LDS histogram acc[Mt], resolving ids
// repeated within a step in rounds through an LDS atomicMin owner (the lowest
// lane, i.e. the earliest position, adds first), so every id's fp32 sum runs
// in (row, slot) order; the positive sums (at most Mt <= 512) are then
// compacted in id order and sorted in registers on 64-bit (score, ~id) keys.
// This replaces a bitonic sort of all g*K (id, position) keys in LDS.
// ----------------------------------------------------------------------------
constexpr int kMergeHistM = 512;

__global__ __launch_bounds__(256) void fta_qblock_merge_hist_kernel(
    const int32_t* __restrict__ idx, const float* __restrict__ scr, int64_t num_slices, int g, int K, int Mt, int W,
    int32_t* __restrict__ out_idx, float* __restrict__ out_scr, int32_t* __restrict__ counts) {
    __shared__ float s_acc[4][kMergeHistM];
    __shared__ int s_owner[4][kMergeHistM];
    __shared__ unsigned long long s_key[4][kMergeHistM];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t slice = (int64_t)blockIdx.x * 4 + wave;
    if (slice >= num_slices) return;  // no workgroup barrier below
    volatile float* acc = s_acc[wave];
    volatile int* owner = s_owner[wave];
    unsigned long long* key = s_key[wave];
    for (int m = lane; m < Mt; m += 64) acc[m] = 0.f;
    fta_wave_sync();
    const int n = g * K;
    const int32_t* ip = idx + slice * (int64_t)n;
    const float* sp = scr + slice * (int64_t)n;
    for (int j0 = 0; j0 < n; j0 += 64) {
        const int j = j0 + lane;
        const int id = (j < n) ? ip[j] : -1;
        const float sc = (j < n) ? sp[j] : 0.f;
        bool pending = id >= 0 && id < Mt;
        while (__ballot(pending) != 0ull) {
            if (pending) owner[id] = 64;
            if (pending) atomicMin(const_cast<int*>(&owner[id]), lane);
            if (pending && owner[id] == lane) {
                acc[id] = __fadd_rn(acc[id], sc);
                pending = false;
            }
        }
    }
    fta_wave_sync();
    // positive sums in id order
    int P = 0;
    for (int base = 0; base < Mt; base += 64) {
        const int m = base + lane;
        const float a = (m < Mt) ? acc[m] : 0.f;
        const bool pos = a > 0.f;
        const unsigned long long mask = __ballot(pos);
        if (pos)
            key[P + __popcll(mask & ((1ull << lane) - 1ull))] =
                ((unsigned long long)__builtin_bit_cast(uint32_t, a) << 32) | (unsigned long long)(0xffffffffu - m);
        P += __popcll(mask);
    }
    int S = 1;
    while (S < P) S <<= 1;
    for (int i = P + lane; i < S; i += 64) key[i] = 0ull;
    fta_wave_sync();
    fta_wave_sort<unsigned long long, true>(key, S, 0ull, lane);  // descending
    const int keep = P < W ? P : W;
    int32_t* oi = out_idx + slice * (int64_t)W;
    float* os = out_scr ? out_scr + slice * (int64_t)W : nullptr;
    for (int p = lane; p < W; p += 64) {
        if (p < keep) {
            const unsigned long long kv = key[p];
            oi[p] = (int)(0xffffffffu - (uint32_t)(kv & 0xffffffffull));
            if (os) os[p] = __builtin_bit_cast(float, (uint32_t)(kv >> 32));
        } else {
            oi[p] = -1;
            if (os) os[p] = 0.f;
        }
    }
    if (counts && lane == 0) counts[slice] = keep;
}

// ----------------------------------------------------------------------------
// Reverse index (reference: flash_topk_attn_v2/sparse_attn_bwd.py:36-76,
// csrc/build_reverse_indices_kernel.cu:6-104).
// Membership bitmap sel[bh][m][qm/32] bit (qm%32) = q-block qm selected KV
// block m.  Bit-OR is order independent, so the lists derived from it (q-block
// ids ascending) are deterministic.
// ----------------------------------------------------------------------------

// Membership bitmap sel[bh][m][qw]: bit (qm & 31) of word qw = qm / 32 is set
// when q-block qm's merged list holds KV block m.  One workgroup per (bh, qw)
// builds that word column for every m in LDS (atomicOr there), a chunk of
// kSelChunk blocks at a time, and writes every word: no global atomics and no
// separate clearing pass.
constexpr int kSelChunk = 8192;

__global__ __launch_bounds__(256) void fta_sel_bitmap_kernel(const int32_t* __restrict__ merged, int QM, int W,
                                                             int M, int QW, uint32_t* __restrict__ sel) {
    __shared__ uint32_t bits[kSelChunk];
    const int64_t bh = blockIdx.x / QW;
    const int qw = (int)(blockIdx.x - bh * QW);
    const int q0 = qw * 32, nq = min(32, QM - q0);
    const int32_t* mp = merged + (bh * QM + q0) * (int64_t)W;
    for (int m0 = 0; m0 < M; m0 += kSelChunk) {
        const int mn = min(kSelChunk, M - m0);
        for (int i = threadIdx.x; i < mn; i += 256) bits[i] = 0u;
        __syncthreads();
        for (int qq = 0; qq < nq; ++qq)
            for (int e = threadIdx.x; e < W; e += 256) {
                const int m = mp[(int64_t)qq * W + e] - m0;
                if (m >= 0 && m < mn) atomicOr(&bits[m], 1u << qq);
            }
        __syncthreads();
        for (int i = threadIdx.x; i < mn; i += 256) sel[(bh * M + m0 + i) * QW + qw] = bits[i];
        __syncthreads();
    }
}

// One wave per (bh, m): ascending q-block list, -1 fill, count.
__global__ __launch_bounds__(64) void fta_reverse_lists_kernel(const uint32_t* __restrict__ sel, int QM, int QW,
                                                                int32_t* __restrict__ rev_idx,
                                                                int32_t* __restrict__ rev_cnt) {
    const int64_t row = blockIdx.x;
    const int lane = threadIdx.x;
    const uint32_t* w = sel + row * QW;
    int32_t* out = rev_idx + row * QM;
    int base = 0;
    for (int w0 = 0; w0 < QW; w0 += 64) {
        const uint32_t bits = (w0 + lane < QW) ? w[w0 + lane] : 0u;
        const int c = __popc(bits);
        int x = c;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const int y = __shfl_up(x, off, 64);
            if (lane >= off) x += y;
        }
        int pos = base + x - c;
        uint32_t bb = bits;
        while (bb) {
            const int j = __ffs(bb) - 1;
            bb &= bb - 1;
            out[pos++] = (w0 + lane) * 32 + j;
        }
        base += __shfl(x, 63, 64);
    }
    for (int i = base + lane; i < QM; i += 64) out[i] = -1;
    if (lane == 0) rev_cnt[row] = base;
}

// Stable descending argsort of counts within each row of length n (one WG per
// row; rank counting keeps ties in ascending index order).
__global__ __launch_bounds__(256) void fta_argsort_desc_rows_kernel(const int32_t* __restrict__ cnt, int n,
                                                                     int32_t* __restrict__ out) {
    __shared__ int c[4096];
    const int64_t row = blockIdx.x;
    const int32_t* in = cnt + row * n;
    for (int i = threadIdx.x; i < n; i += 256) c[i] = in[i];
    __syncthreads();
    for (int i = threadIdx.x; i < n; i += 256) {
        const int ci = c[i];
        int rank = 0;
        for (int j = 0; j < n; ++j) {
            const int cj = c[j];
            rank += (cj > ci) || (cj == ci && j < i);
        }
        out[row * n + rank] = i;
    }
}

// Launch order of the dK/dV workgroups of one (b, K/V head): the KV blocks by
// the number of q-blocks that selected them, most first (ties: ascending block
// id), from the membership bitmap of the group's first query head.  Longest
// first shortens the tail of each XCD's queue, and under dense selections the
// WGs that start together walk q-block lists of the same length and density,
// so they stay at nearby q-blocks and share their Q / dO in L2.  head_work
// receives the head's total (selections plus one setup step per block) for
// fta_head_balance_kernel.
__global__ __launch_bounds__(256) void fta_kv_order_kernel(const uint32_t* __restrict__ sel, int M, int QW, int H,
                                                           int G, int slice_blocks, int32_t* __restrict__ order,
                                                           int32_t* __restrict__ head_work) {
    // WG (b, K/V head, slice): counts every block's selections (coalesced reads
    // of the bitmap rows, LDS atomics), then ranks the blocks of its slice of
    // slice_blocks (256 or 1024: one to four per thread).  Each slice reads the
    // head's whole bitmap: small heads rank in slices of 256 (the ranking, O(M)
    // per block, dominates), heads of more than 1024 blocks in slices of 1024
    // (four times fewer bitmap re-reads).
    __shared__ uint32_t key[4096];
    __shared__ int s_work;
    const int64_t rk = blockIdx.x;               // (b, K/V head)
    const int slice = blockIdx.y;
    const int64_t bh = (rk / (H / G)) * H + (rk % (H / G)) * G;  // its first query head
    const uint32_t* rows = sel + bh * (int64_t)M * QW;
    for (int m = threadIdx.x; m < M; m += 256) key[m] = 0xffffffffu;
    if (threadIdx.x == 0) s_work = M;  // one setup step per block
    __syncthreads();
    const int64_t nw = (int64_t)M * QW;
    int cw = 0;
    for (int64_t i0 = threadIdx.x; i0 < nw; i0 += 8 * 256) {
        uint32_t wv[8];  // eight loads in flight before any use
#pragma unroll
        for (int u = 0; u < 8; ++u) wv[u] = (i0 + u * 256 < nw) ? rows[i0 + u * 256] : 0u;
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int c = __builtin_popcount(wv[u]);
            if (c) atomicSub(&key[(i0 + u * 256) / QW], (uint32_t)c);
            cw += c;
        }
    }
    atomicAdd(&s_work, cw);
    __syncthreads();
    if (slice == 0 && threadIdx.x == 0) head_work[rk] = s_work;
    for (int u = 0; u < slice_blocks / 256; ++u) {
        const int i = slice * slice_blocks + u * 256 + threadIdx.x;
        if (i < M) {
            const uint32_t ki = key[i];
            int rank = 0;
            for (int j = 0; j < M; ++j) {
                const uint32_t kj = key[j];
                rank += (kj < ki) || (kj == ki && j < i);
            }
            order[rk * M + rank] = i;
        }
    }
}

// XCD placement of the dK/dV heads.  The WGs of head position p run on XCD
// p / (n / 8) (fta_xcd_remap gives each XCD a contiguous range of the grid), so
// heads of unequal total work (head_work: selection counts plus setup) leave
// some XCDs busy after others have drained.  Greedy longest-first placement of
// the heads into 8 bins of n / 8 heads each evens the XCD totals; perm[p] is
// the head at position p (bins in XCD order, heaviest first within a bin).
// n not a multiple of 8, or above 4096 heads: identity.
// With `part` set, each head's work is first formed from its partial counts:
// head_work[i] = base + scale * sum_j part[i][j] (j < nparts).
__global__ __launch_bounds__(256) void fta_head_balance_kernel(int32_t* __restrict__ head_work,
                                                               const int32_t* __restrict__ part, int nparts,
                                                               int base, int scale, int n,
                                                               int32_t* __restrict__ perm) {
    __shared__ int w[4096];
    __shared__ int by_rank[4096];
    if (part != nullptr) {
        for (int i = threadIdx.x; i < n; i += 256) {
            int c = 0;
            for (int j = 0; j < nparts; ++j) c += part[(int64_t)i * nparts + j];
            head_work[i] = base + scale * c;
        }
        __syncthreads();
    }
    if (n % 8 != 0 || n > 4096) {
        for (int i = threadIdx.x; i < n; i += 256) perm[i] = i;
        return;
    }
    for (int i = threadIdx.x; i < n; i += 256) w[i] = head_work[i];
    __syncthreads();
    for (int i = threadIdx.x; i < n; i += 256) {
        const int wi = w[i];
        int rank = 0;
        for (int j = 0; j < n; ++j) rank += (w[j] > wi) || (w[j] == wi && j < i);
        by_rank[rank] = i;
    }
    __syncthreads();
    // greedy placement by the first wave: lane x < 8 keeps bin x's load and fill
    if (threadIdx.x < 64) {
        const int x = threadIdx.x;
        const int cap = n / 8;
        long long load = 0;
        int fill = 0;
        for (int r = 0; r < n; ++r) {
            const int hd = by_rank[r];
            // the open bin with the least load (ties: lowest bin)
            long long key = (x < 8 && fill < cap) ? load * 8 + x : 0x7fffffffffffffffll;
#pragma unroll
            for (int off = 4; off > 0; off >>= 1) {
                const long long o = __shfl_xor(key, off, 8);
                key = o < key ? o : key;
            }
            const int best = (int)(key & 7);
            if (x == best) {
                perm[best * cap + fill] = hd;
                ++fill;
                load += w[hd];
            }
        }
    }
}

// Work of each (b, h) for the forward / dQ head placement: its valid merged
// entries (KV blocks selected by its q-blocks) plus one setup step per four
// q-blocks.  WG (bh, j) counts q-block rows j, j + kHeadParts, ... into
// part[bh][j]; fta_head_balance_kernel adds the parts.  (Counting every fourth
// row only placed the C3 heads 5% worse.)
constexpr int kHeadParts = 64;
// Union-based work of each (b, h) for the forward placement.  Group gi holds the
// qpg consecutive q-blocks of one forward workgroup; WG (bh, j) takes groups j,
// j + kHeadParts, ...  A group costs the size of the union of its q-blocks'
// lists (the chunks its workgroup walks) plus `setup` chunk-steps.  M <= 4096.
__global__ __launch_bounds__(256) void fta_head_work_union_kernel(const int32_t* __restrict__ merged, int QM, int W,
                                                                  int M, int qpg, int setup,
                                                                  int32_t* __restrict__ part) {
    __shared__ uint32_t bits[128];
    __shared__ int s_u;
    const int tid = threadIdx.x;
    const int bh = blockIdx.x / kHeadParts, j = blockIdx.x % kHeadParts;
    const int ngroups = (QM + qpg - 1) / qpg;
    int work = 0;
    for (int gi = j; gi < ngroups; gi += kHeadParts) {
        if (tid < 128) bits[tid] = 0u;
        if (tid == 0) s_u = 0;
        __syncthreads();
        const int q0 = gi * qpg, q1 = min(QM, q0 + qpg);
        const int32_t* rows = merged + ((int64_t)bh * QM + q0) * W;
        const int n = (q1 - q0) * W;
        for (int e = tid; e < n; e += 256) {
            const int m = rows[e];
            if (m >= 0 && m < M) atomicOr(&bits[m >> 5], 1u << (m & 31));
        }
        __syncthreads();
        int c = (tid < 128) ? __popc(bits[tid]) : 0;
        for (int off = 32; off > 0; off >>= 1) c += __shfl_xor(c, off, 64);
        if ((tid & 63) == 0 && c) atomicAdd(&s_u, c);
        __syncthreads();
        work += s_u + setup;
        __syncthreads();
    }
    if (tid == 0) part[blockIdx.x] = work;
}

__global__ __launch_bounds__(256) void fta_head_work_merged_kernel(const int32_t* __restrict__ merged, int QM, int W,
                                                                   int M, int32_t* __restrict__ part) {
    __shared__ int s_work;
    if (threadIdx.x == 0) s_work = 0;
    __syncthreads();
    const int bh = blockIdx.x / kHeadParts, j = blockIdx.x % kHeadParts;
    int c = 0;
    for (int qb = j; qb < QM; qb += kHeadParts) {
        const int32_t* row = merged + ((int64_t)bh * QM + qb) * W;
        for (int i = threadIdx.x; i < W; i += 256) {
            const int m = row[i];
            c += (m >= 0 && m < M);
        }
    }
    for (int off = 32; off > 0; off >>= 1) c += __shfl_xor(c, off, 64);
    if ((threadIdx.x & 63) == 0) atomicAdd(&s_work, c);
    __syncthreads();
    if (threadIdx.x == 0) part[blockIdx.x] = s_work;
}

// Global stable descending sort of counts (reference: sort_by_count_cuda.py:33-67):
// rank_i = #{j : c_j > c_i} + #{j < i : c_j == c_i}.
__global__ __launch_bounds__(256) void fta_sort_by_count_kernel(const int32_t* __restrict__ cnt, int n,
                                                                 int32_t* __restrict__ sorted_cnt,
                                                                 int32_t* __restrict__ sorted_ids) {
    __shared__ int tile[2048];
    const int i = blockIdx.x * 256 + threadIdx.x;
    const int ci = (i < n) ? cnt[i] : 0;
    int rank = 0;
    for (int t0 = 0; t0 < n; t0 += 2048) {
        __syncthreads();
        for (int j = threadIdx.x; j < 2048; j += 256) tile[j] = (t0 + j < n) ? cnt[t0 + j] : -2147483647 - 1;
        __syncthreads();
        const int lim = (n - t0 < 2048) ? n - t0 : 2048;
        for (int j = 0; j < lim; ++j) {
            const int cj = tile[j];
            rank += (cj > ci) || (cj == ci && t0 + j < i);
        }
    }
    if (i < n) {
        sorted_cnt[rank] = ci;
        sorted_ids[rank] = i;
    }
}

// ----------------------------------------------------------------------------
// delta[bh][n] = sum_d O * dO in fp32 (reference: sparse_attn_bwd.py:12-33).
// ----------------------------------------------------------------------------
template <int DT>
__global__ __launch_bounds__(256) void fta_delta_kernel(const uint16_t* __restrict__ o, int64_t o_sb, int64_t o_sh,
                                                        int64_t o_sn, const uint16_t* __restrict__ dout,
                                                        int64_t d_sb, int64_t d_sh, int64_t d_sn, int B, int H,
                                                        int N, int D, float* __restrict__ delta) {
    // 16 lanes per (b, n, h) row: each pass reads 256 contiguous bytes of o and
    // of dO per row (8 elements per lane); partial sums meet in a 16-lane tree
    using E = Elem<DT>;
    const int64_t row = ((int64_t)blockIdx.x * 256 + threadIdx.x) >> 4;  // (b, n, h)
    const int sub = threadIdx.x & 15;
    const bool valid = row < (int64_t)B * N * H;
    float acc = 0.f;
    int b = 0, n = 0, h = 0;
    if (valid) {
        h = (int)(row % H);
        const int64_t bn = row / H;
        n = (int)(bn % N);
        b = (int)(bn / N);
        const uint16_t* op = o + b * o_sb + h * o_sh + (int64_t)n * o_sn;
        const uint16_t* dp = dout + b * d_sb + h * d_sh + (int64_t)n * d_sn;
        for (int d = sub * 8; d < D; d += 128) {
            const uint4 a = *reinterpret_cast<const uint4*>(op + d);
            const uint4 c = *reinterpret_cast<const uint4*>(dp + d);
            const uint32_t av[4] = {a.x, a.y, a.z, a.w}, cv[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                acc = fmaf(E::to_f32((uint16_t)(av[e] & 0xffffu)), E::to_f32((uint16_t)(cv[e] & 0xffffu)), acc);
                acc = fmaf(E::to_f32((uint16_t)(av[e] >> 16)), E::to_f32((uint16_t)(cv[e] >> 16)), acc);
            }
        }
    }
#pragma unroll
    for (int w = 8; w >= 1; w >>= 1) acc += __shfl_xor(acc, w, 16);
    if (valid && sub == 0) delta[((int64_t)b * H + h) * N + n] = acc;
}


// ----------------------------------------------------------------------------
// q-block union (reference V1: flash_topk_attn/attention.py:23-138).  One
// wave per (b, h, q-block): the g*K ids of the block's query rows (rows
// outside [0, N) under the virtual q padding contribute -1) are sorted
// ascending (bitonic in registers up to 512 ids, else in the wave's LDS slab;
// P = next pow2 of g*K, -1 mapped past every id), then the first copy of each non-negative id is compacted to the front of
// the P-wide output row; the rest of the row is -1 and counts = #unique ids.
// ----------------------------------------------------------------------------
__global__ __launch_bounds__(256) void fta_qblock_union_kernel(const int32_t* __restrict__ idx, int N, int K,
                                                               int g, int q_pad_head, int QM, int P,
                                                               int64_t slices, int32_t* __restrict__ merged,
                                                               int32_t* __restrict__ counts) {
    extern __shared__ __align__(16) unsigned char smem[];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, wpb = blockDim.x >> 6;
    const int64_t slice = (int64_t)blockIdx.x * wpb + wave;
    if (slice >= slices) return;
    uint32_t* key = reinterpret_cast<uint32_t*>(smem) + (size_t)wave * P;
    const int64_t bh = slice / QM;
    const int qm = (int)(slice - bh * QM);
    const int n = g * K;
    const int row0 = qm * g - q_pad_head;
    const int32_t* src = idx + bh * (int64_t)N * K;
    for (int i = lane; i < P; i += 64) {
        uint32_t v = 0x7fffffffu;  // sorts after every id
        if (i < n) {
            const int r = row0 + i / K;
            if (r >= 0 && r < N) {
                const int id = src[(int64_t)r * K + (i - (i / K) * K)];
                if (id >= 0) v = (uint32_t)id;
            }
        }
        key[i] = v;
    }
    fta_wave_sync();
    fta_wave_sort<uint32_t, false>(key, P, 0x7fffffffu, lane);
    // the first copy of each id, compacted in ascending order
    int32_t* out = merged + slice * (int64_t)P;
    int total = 0;
    for (int r0 = 0; r0 < P; r0 += 64) {
        const int i = r0 + lane;
        const uint32_t v = (i < P) ? key[i] : 0x7fffffffu;
        const bool fresh = v != 0x7fffffffu && (i == 0 || v != key[i - 1]);
        const unsigned long long mask = __ballot(fresh);
        if (fresh) out[total + __popcll(mask & ((1ull << lane) - 1ull))] = (int32_t)v;
        total += __popcll(mask);
    }
    for (int i = total + lane; i < P; i += 64) out[i] = -1;
    if (lane == 0) counts[slice] = total;
}

namespace fta {

int launch_sel_bitmap(const int32_t* merged, int BH, int QM, int W, int M, uint32_t* sel, hipStream_t st) {
    const int QW = (QM + 31) / 32;
    if ((int64_t)BH * QW == 0 || M <= 0) return FTA_OK;
    hipLaunchKernelGGL(fta_sel_bitmap_kernel, dim3((unsigned)((int64_t)BH * QW)), dim3(256), 0, st, merged, QM, W,
                       M, QW, sel);
    return check_launch("fta_sel_bitmap_kernel");
}

int launch_kv_order(const uint32_t* sel, int B, int H, int Hk, int M, int QW, int32_t* order, int32_t* head_work,
                    int32_t* head_perm, hipStream_t st) {
    if (M <= 0 || B * Hk == 0) return FTA_OK;
    const int slice = (M > 1024) ? 1024 : 256;
    hipLaunchKernelGGL(fta_kv_order_kernel, dim3((unsigned)(B * Hk), (unsigned)((M + slice - 1) / slice)), dim3(256), 0,
                       st, sel, M, QW, H, H / Hk, slice, order, head_work);
    int rc = check_launch("fta_kv_order_kernel");
    if (rc != FTA_OK) return rc;
    hipLaunchKernelGGL(fta_head_balance_kernel, dim3(1), dim3(256), 0, st, head_work, nullptr, 0, 0, 1, B * Hk,
                       head_perm);
    return check_launch("fta_head_balance_kernel");
}

int launch_head_order_merged(const int32_t* merged, int BH, int QM, int W, int M, int qpg, int32_t* head_work,
                             int32_t* head_perm, hipStream_t st) {
    if (BH <= 0) return FTA_OK;
    // part sums after head_work and head_perm: [BH][kHeadParts]
    int32_t* part = head_perm + BH;
    int rc;
    if (M <= 4096) {
        hipLaunchKernelGGL(fta_head_work_union_kernel, dim3((unsigned)(BH * kHeadParts)), dim3(256), 0, st, merged,
                           QM, W, M, qpg, 3, part);
        if ((rc = check_launch("fta_head_work_union_kernel")) != FTA_OK) return rc;
        hipLaunchKernelGGL(fta_head_balance_kernel, dim3(1), dim3(256), 0, st, head_work, part, kHeadParts, 0, 1, BH,
                           head_perm);
        return check_launch("fta_head_balance_kernel");
    }
    hipLaunchKernelGGL(fta_head_work_merged_kernel, dim3((unsigned)(BH * kHeadParts)), dim3(256), 0, st, merged, QM,
                       W, M, part);
    rc = check_launch("fta_head_work_merged_kernel");
    if (rc != FTA_OK) return rc;
    hipLaunchKernelGGL(fta_head_balance_kernel, dim3(1), dim3(256), 0, st, head_work, part, kHeadParts, QM / 4, 1, BH,
                       head_perm);
    return check_launch("fta_head_balance_kernel");
}
}  // namespace fta

namespace fta {
// One-wave-per-slice merge when g*K <= 4096 (LDS: 16 B per padded entry per
// wave), the histogram kernel otherwise.
int launch_qblock_merge(const int32_t* idx, const float* scr, int64_t num_slices, int g, int K, int Mt,
                        const int32_t* max_id, int W, int32_t* out_idx, float* out_scr, int32_t* counts,
                        hipStream_t st) {
    const int64_t n = (int64_t)g * K;
    if (n >= 1 && n <= 32) {
        const int64_t blocks = (num_slices + 255) / 256;
        if (n <= 16)
            hipLaunchKernelGGL(fta_qblock_merge_lane_kernel<16>, dim3((unsigned)blocks), dim3(256), 0, st, idx, scr,
                               num_slices, (int)n, Mt, max_id, W, out_idx, out_scr, counts);
        else
            hipLaunchKernelGGL(fta_qblock_merge_lane_kernel<32>, dim3((unsigned)blocks), dim3(256), 0, st, idx, scr,
                               num_slices, (int)n, Mt, max_id, W, out_idx, out_scr, counts);
        return check_launch("fta_qblock_merge_lane_kernel");
    }
    if (max_id == nullptr && n > 512 && Mt <= kMergeHistM) {
        // many entries over few blocks: histogram per wave instead of a sort of every entry
        const int64_t blocks = (num_slices + 3) / 4;
        hipLaunchKernelGGL(fta_qblock_merge_hist_kernel, dim3((unsigned)blocks), dim3(256), 0, st, idx, scr,
                           num_slices, g, K, Mt, W, out_idx, out_scr, counts);
        return check_launch("fta_qblock_merge_hist_kernel");
    }
    if (n >= 1 && n <= kMergeWaveMax) {
        int NP = 1;
        while (NP < n) NP <<= 1;
        const int wpb = (NP <= 1024) ? 4 : (NP <= 2048) ? 2 : 1;
        const int64_t blocks = (num_slices + wpb - 1) / wpb;
        hipLaunchKernelGGL(fta_qblock_merge_wave_kernel, dim3((unsigned)blocks), dim3(64 * wpb),
                           (size_t)wpb * NP * 16, st, idx, scr, num_slices, g, K, NP, Mt, max_id, W, out_idx,
                           out_scr, counts);
        return check_launch("fta_qblock_merge_wave_kernel");
    }
    hipLaunchKernelGGL(fta_qblock_merge_kernel, dim3((unsigned)num_slices), dim3(256), 0, st, idx, scr, g, K, Mt,
                       max_id, W, out_idx, out_scr, counts);
    return check_launch("fta_qblock_merge_kernel");
}
}  // namespace fta

extern "C" {

int fta_qblock_merge(const int32_t* topk_indices, const float* topk_scores, int64_t num_slices, int q_block_size,
                     int k_per_query, int num_score_blocks, int qblock_topk, int32_t* merged_indices,
                     float* merged_scores, int32_t* counts, void* stream) {
    FTA_TRY_BEGIN
    if (num_slices < 0 || num_slices > 0x7fffffff) return fta::arg_error("qblock_merge: bad slice count");
    if (q_block_size <= 0 || k_per_query < 0) return fta::arg_error("qblock_merge: bad q_block_size / K");
    if (num_score_blocks <= 0) return fta::arg_error("num_score_blocks must be positive");
    if (num_score_blocks > 4096) return fta::unsupported("num_score_blocks exceeds block sort limit 4096");
    if (qblock_topk <= 0) return fta::arg_error("qblock_topk must be positive");
    if (num_slices == 0) return FTA_OK;
    return fta::launch_qblock_merge(topk_indices, topk_scores, num_slices, q_block_size, k_per_query,
                                    num_score_blocks, nullptr, qblock_topk, merged_indices, merged_scores, counts,
                                    (hipStream_t)stream);
    FTA_TRY_END
}

int fta_qblock_merge_maxid(const int32_t* topk_indices, const float* topk_scores, int64_t num_slices,
                           int q_block_size, int k_per_query, const int32_t* max_index, int qblock_topk,
                           int32_t* merged_indices, float* merged_scores, int32_t* counts, void* stream) {
    FTA_TRY_BEGIN
    if (num_slices < 0 || num_slices > 0x7fffffff) return fta::arg_error("qblock_merge: bad slice count");
    if (q_block_size <= 0 || k_per_query < 0) return fta::arg_error("qblock_merge: bad q_block_size / K");
    if (max_index == nullptr) return fta::arg_error("qblock_merge: max_index is NULL");
    if (qblock_topk <= 0) return fta::arg_error("qblock_topk must be positive");
    if (num_slices == 0) return FTA_OK;
    return fta::launch_qblock_merge(topk_indices, topk_scores, num_slices, q_block_size, k_per_query, 0,
                                    max_index, qblock_topk, merged_indices, merged_scores, counts,
                                    (hipStream_t)stream);
    FTA_TRY_END
}

int fta_qblock_union(const int32_t* topk_indices, int BH, int N, int K, int q_block_size, int q_pad_head,
                     int q_pad_tail, int s_max, int32_t* merged_indices, int32_t* counts, void* stream) {
    FTA_TRY_BEGIN
    if (BH < 0 || N < 0 || K < 0) return fta::arg_error("qblock_union: negative dims");
    if (q_block_size <= 0) return fta::arg_error("qblock_union: q_block_size must be positive");
    if (q_pad_head < 0 || q_pad_tail < 0 || q_pad_head >= q_block_size || q_pad_tail >= q_block_size)
        return fta::arg_error("qblock_union: q padding must each be in [0, q_block_size)");
    const int64_t np = (int64_t)q_pad_head + N + q_pad_tail;
    if (np % q_block_size != 0) return fta::arg_error("qblock_union: q_pad_head + N + q_pad_tail not divisible");
    const int64_t n = (int64_t)q_block_size * K;
    if (s_max <= 0 || (s_max & (s_max - 1)) != 0 || s_max < n)
        return fta::arg_error("qblock_union: s_max must be a power of two >= q_block_size * K");
    if (s_max > kUnionMax) return fta::unsupported("qblock_union: q_block_size * K exceeds 8192");
    const int QM = (int)(np / q_block_size);
    const int64_t slices = (int64_t)BH * QM;
    if (slices > 0x7fffffff) return fta::arg_error("qblock_union: too many q-blocks");
    if (slices == 0) return FTA_OK;
    if (!topk_indices && n > 0 && N > 0) return fta::arg_error("qblock_union: topk_indices is NULL");
    if (!merged_indices || !counts) return fta::arg_error("qblock_union: null output");
    // one wave per slice (LDS: s_max ids per wave, at most 32 KB per workgroup)
    const int wpb = (s_max <= 2048) ? 4 : (s_max <= 4096) ? 2 : 1;
    hipLaunchKernelGGL(fta_qblock_union_kernel, dim3((unsigned)((slices + wpb - 1) / wpb)), dim3(64 * wpb),
                       (size_t)wpb * s_max * sizeof(int), (hipStream_t)stream, topk_indices, N, K, q_block_size,
                       q_pad_head, QM, s_max, slices, merged_indices, counts);
    return fta::check_launch("fta_qblock_union_kernel");
    FTA_TRY_END
}

size_t fta_build_reverse_indices_workspace_size(int B, int H, int QM, int M) {
    return fta::align_up((size_t)B * H * M * ((QM + 31) / 32) * sizeof(uint32_t));
}

int fta_build_reverse_indices(const int32_t* merged_indices, const int32_t* counts, int B, int H, int QM, int W,
                              int M, int32_t* reverse_indices, int32_t* reverse_counts, int32_t* sorted_kv_indices,
                              void* workspace, size_t workspace_bytes, void* stream) {
    FTA_TRY_BEGIN
    (void)counts;  // membership is read from the -1 padded lists directly
    if (B <= 0 || H <= 0 || QM <= 0 || W <= 0 || M <= 0) return fta::arg_error("build_reverse_indices: bad dims");
    if (M > 4096) return fta::unsupported("build_reverse_indices: M exceeds 4096");
    if (workspace_bytes < fta_build_reverse_indices_workspace_size(B, H, QM, M))
        return fta::arg_error("build_reverse_indices: workspace too small");
    hipStream_t st = (hipStream_t)stream;
    uint32_t* sel = (uint32_t*)workspace;
    int rc = fta::launch_sel_bitmap(merged_indices, B * H, QM, W, M, sel, st);
    if (rc != FTA_OK) return rc;
    const int QW = (QM + 31) / 32;
    hipLaunchKernelGGL(fta_reverse_lists_kernel, dim3((unsigned)((int64_t)B * H * M)), dim3(64), 0, st, sel, QM, QW,
                       reverse_indices, reverse_counts);
    rc = fta::check_launch("fta_reverse_lists_kernel");
    if (rc != FTA_OK) return rc;
    if (sorted_kv_indices) {
        hipLaunchKernelGGL(fta_argsort_desc_rows_kernel, dim3((unsigned)(B * H)), dim3(256), 0, st, reverse_counts,
                           M, sorted_kv_indices);
        rc = fta::check_launch("fta_argsort_desc_rows_kernel");
    }
    return rc;
    FTA_TRY_END
}

int fta_sort_by_count(const int32_t* reverse_counts, int64_t total, int32_t* sorted_counts, int32_t* sorted_ids,
                      void* stream) {
    FTA_TRY_BEGIN
    if (total < 0 || total > 0x7fffffff) return fta::arg_error("sort_by_count: bad size");
    if (total == 0) return FTA_OK;
    hipLaunchKernelGGL(fta_sort_by_count_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                       (hipStream_t)stream, reverse_counts, (int)total, sorted_counts, sorted_ids);
    return fta::check_launch("fta_sort_by_count_kernel");
    FTA_TRY_END
}

int fta_preprocess_delta(const void* o, const int64_t* o_strides, const void* dout, const int64_t* do_strides,
                         int dtype, int B, int H, int N, int D, float* delta, void* stream) {
    FTA_TRY_BEGIN
    if (B <= 0 || H <= 0 || N <= 0 || D <= 0 || D % 8) return fta::arg_error("preprocess_delta: bad dims");
    const int64_t n = (int64_t)B * N * H;
    if (n > ((int64_t)1 << 35)) return fta::unsupported("preprocess_delta: too many rows");
    const unsigned grid = (unsigned)((n * 16 + 255) / 256);  // 16 lanes per row
    hipStream_t st = (hipStream_t)stream;
    if (dtype == FTA_DTYPE_BF16)
        hipLaunchKernelGGL((fta_delta_kernel<FTA_DTYPE_BF16>), dim3(grid), dim3(256), 0, st, (const uint16_t*)o,
                           o_strides[0], o_strides[1], o_strides[2], (const uint16_t*)dout, do_strides[0],
                           do_strides[1], do_strides[2], B, H, N, D, delta);
    else if (dtype == FTA_DTYPE_F16)
        hipLaunchKernelGGL((fta_delta_kernel<FTA_DTYPE_F16>), dim3(grid), dim3(256), 0, st, (const uint16_t*)o,
                           o_strides[0], o_strides[1], o_strides[2], (const uint16_t*)dout, do_strides[0],
                           do_strides[1], do_strides[2], B, H, N, D, delta);
    else
        return fta::arg_error("preprocess_delta: dtype must be bf16 or fp16");
    return fta::check_launch("fta_delta_kernel");
    FTA_TRY_END
}

}  // extern "C"
