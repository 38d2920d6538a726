// Host-side helpers shared by the extern "C" entry points.
// Every entry point returns an int status (FTA_OK / FTA_ERR_*) and never lets a
// C++ exception cross the ABI; the last error message is kept per thread and
// returned by fta_last_error().
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "fta_common.h"

namespace fta {

void set_error(const std::string& msg);

inline int arg_error(const char* msg) {
    set_error(msg);
    return FTA_ERR_ARG;
}
inline int unsupported(const char* msg) {
    set_error(msg);
    return FTA_ERR_UNSUPPORTED;
}

inline int check_launch(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_error(std::string(what) + ": " + hipGetErrorString(e));
        return FTA_ERR_HIP;
    }
    return FTA_OK;
}

inline size_t align_up(size_t x, size_t a = 256) { return (x + a - 1) / a * a; }

// Head dims the kernels are instantiated for; inputs with a smaller D are
// zero-extended on load (the reference pads with F.pad to the same set,
// flash_topk_attn_v2/sparse_attn.py:349-373, block_score_cuda.py:112-132).
inline int kernel_head_dim(int D) {
    static const int kDims[] = {32, 64, 96, 128, 160, 256};
    for (int d : kDims)
        if (d >= D) return d;
    return -1;
}

inline int check_score_args(int B, int H, int N, int D, int bsz, int pad_head, int pad_tail, int* M) {
    if (B <= 0 || H <= 0 || N <= 0 || D <= 0) return arg_error("block_score: dims must be positive");
    if (bsz <= 0) return arg_error("block_score: score_block_size must be positive");
    if (pad_head < 0 || pad_tail < 0) return arg_error("padding must be non-negative (pad_head, pad_tail)");
    if (pad_head >= bsz || pad_tail >= bsz) return arg_error("padding must each be < score_block_size");
    const int64_t np = (int64_t)pad_head + N + pad_tail;
    if (np % bsz != 0) return arg_error("pad_head + N + pad_tail must be divisible by score_block_size");
    *M = (int)(np / bsz);
    return FTA_OK;
}

}  // namespace fta

#define FTA_TRY_BEGIN try {
#define FTA_TRY_END                                 \
    }                                               \
    catch (const std::exception& ex) {              \
        fta::set_error(ex.what());                  \
        return FTA_ERR_HIP;                         \
    }                                               \
    catch (...) {                                   \
        fta::set_error("unknown C++ exception");    \
        return FTA_ERR_HIP;                         \
    }
