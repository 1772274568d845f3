// sdpa_checks.h -- argument checks and status messages of the Sdpa /
// SdpaGrad C ABIs, shared by the GPU library (sdpa_capi.hip, sdpa_hip_*) and
// the host-kernel library (sdpa_host.cc, sdpa_cpu_*), so that both report
// the reference's errors in the reference's order with the same messages.
// Host code only; status codes are those of include/sdpa_hip.h.
#pragma once

#include <stdint.h>

#include "sdpa_hip.h"

namespace sdpa {

inline const char* status_message(int status) {
    switch (status) {
        case SDPA_OK: return "OK";
        case SDPA_ERR_SEED_NOT_SCALAR: return "seed must be scalar";
        case SDPA_ERR_OFFSET_NOT_SCALAR: return "offset must be scalar";
        case SDPA_ERR_K_BATCH: return "K batch size mismatch";
        case SDPA_ERR_K_FEATURE: return "K feature size mismatch";
        case SDPA_ERR_V_BATCH: return "V batch size mismatch";
        case SDPA_ERR_V_SEQ: return "V seq size mismatch";
        case SDPA_ERR_O_BATCH: return "O batch size mismatch";
        case SDPA_ERR_O_SEQ: return "O seq size mismatch";
        case SDPA_ERR_O_FEATURE: return "O feature size mismatch";
        case SDPA_ERR_DO_BATCH: return "dO batch size mismatch";
        case SDPA_ERR_DO_SEQ: return "dO seq size mismatch";
        case SDPA_ERR_DO_FEATURE: return "dO feature size mismatch";
        case SDPA_ERR_S_BATCH: return "S batch size mismatch";
        case SDPA_ERR_S_SEQ: return "S seq size mismatch";
        case SDPA_ERR_CAUSAL_SEQ: return "seq size Q != K while causal_mask = True";
        case SDPA_ERR_FEATURE_TOO_LARGE:
            return "CUDA kernel does not support feature size over 128. Set smaller feature size or "
                   "use more heads";
        case SDPA_ERR_RANK: return "Shape must be rank 3";
        case SDPA_ERR_DTYPE: return "dtype must be float16 or float32";
        case SDPA_ERR_NEGATIVE_DIM: return "tensor dimensions must be non-negative";
        case SDPA_ERR_NULL_POINTER: return "null pointer for a non-empty tensor";
        case SDPA_ERR_DROPOUT_RANGE: return "dropout must not be 1 (the kept elements would be scaled by 1 / (1 - p))";
        case SDPA_ERR_WORKSPACE: return "backward workspace is too small";
        case SDPA_ERR_HIP: return "HIP runtime error";
        case SDPA_ERR_SCRATCH_LIMIT:
            return "B * S_q exceeds the static scratch of sdpa_hip_bwd_noalloc (2097152 query rows)";
        case SDPA_ERR_DS_PATH:
            return "the dS path of the backward needs float16, a feature size over 64, 16-byte aligned tensors "
                   "and a workspace of sdpa_hip_bwd_workspace_bytes_ds bytes";
        default: return "unknown sdpa status";
    }
}

// Sdpa: rank of every input, scalar seed / offset, then the reference's
// OP_REQUIRES order (sdpa/sdpa_ops.cc:22-25, sdpa/sdpa_cpu.cc:37-69).
inline int check_fwd_shapes(int q_rank, const int64_t* q, int k_rank, const int64_t* k, int v_rank,
                            const int64_t* v, int seed_rank, int offset_rank, int causal_mask) {
    if (q_rank != 3 || k_rank != 3 || v_rank != 3) return SDPA_ERR_RANK;  // sdpa_ops.cc:22-25
    if (seed_rank != 0) return SDPA_ERR_SEED_NOT_SCALAR;                  // sdpa_cpu.cc:37-40
    if (offset_rank != 0) return SDPA_ERR_OFFSET_NOT_SCALAR;
    if (k[0] != q[0]) return SDPA_ERR_K_BATCH;  // sdpa_cpu.cc:51-58
    if (k[2] != q[2]) return SDPA_ERR_K_FEATURE;
    if (v[0] != q[0]) return SDPA_ERR_V_BATCH;
    if (v[1] != k[1]) return SDPA_ERR_V_SEQ;
    if (causal_mask && q[1] != k[1]) return SDPA_ERR_CAUSAL_SEQ;      // :60-64
    if ((q[2] > v[2] ? q[2] : v[2]) > 128) return SDPA_ERR_FEATURE_TOO_LARGE;  // :66-69
    return SDPA_OK;
}

// SdpaGrad (sdpa/sdpa_ops.cc:55-57, sdpa/sdpa_cpu.cc:116-168).
inline int check_bwd_shapes(int q_rank, const int64_t* q, int k_rank, const int64_t* k, int v_rank,
                            const int64_t* v, int o_rank, const int64_t* o, int stats_rank,
                            const int64_t* st, int do_rank, const int64_t* d_o, int seed_rank,
                            int offset_rank, int causal_mask) {
    if (q_rank != 3 || k_rank != 3 || v_rank != 3) return SDPA_ERR_RANK;  // sdpa_ops.cc:55-57
    if (seed_rank != 0) return SDPA_ERR_SEED_NOT_SCALAR;                  // sdpa_cpu.cc:116-119
    if (offset_rank != 0) return SDPA_ERR_OFFSET_NOT_SCALAR;
    // The reference indexes dim_size(0..2) of out/do and (0..1) of stats;
    // a tensor of lower rank has no such dimension and fails the same check.
    auto dim = [](int rank, const int64_t* s, int i) -> int64_t { return i < rank ? s[i] : -1; };
    if (k[0] != q[0]) return SDPA_ERR_K_BATCH;  // sdpa_cpu.cc:130-133
    if (k[2] != q[2]) return SDPA_ERR_K_FEATURE;
    if (v[0] != q[0]) return SDPA_ERR_V_BATCH;  // :135-138
    if (v[1] != k[1]) return SDPA_ERR_V_SEQ;
    if (dim(o_rank, o, 0) != q[0]) return SDPA_ERR_O_BATCH;  // :140-145
    if (dim(o_rank, o, 1) != q[1]) return SDPA_ERR_O_SEQ;
    if (dim(o_rank, o, 2) != v[2]) return SDPA_ERR_O_FEATURE;
    if (dim(do_rank, d_o, 0) != q[0]) return SDPA_ERR_DO_BATCH;  // :147-152
    if (dim(do_rank, d_o, 1) != q[1]) return SDPA_ERR_DO_SEQ;
    if (dim(do_rank, d_o, 2) != v[2]) return SDPA_ERR_DO_FEATURE;
    if (dim(stats_rank, st, 0) != q[0]) return SDPA_ERR_S_BATCH;  // :154-157
    if (dim(stats_rank, st, 1) != q[1]) return SDPA_ERR_S_SEQ;
    if (causal_mask && q[1] != k[1]) return SDPA_ERR_CAUSAL_SEQ;  // :159-163
    if ((q[2] > v[2] ? q[2] : v[2]) > 128) return SDPA_ERR_FEATURE_TOO_LARGE;  // :165-168
    return SDPA_OK;
}

}  // namespace sdpa
