// sdpa_params.h -- kernel argument blocks shared by the host launchers and the
// HIP kernels.  Every tensor is dense row-major [B, S, D] (reference indexing
// (batch_offset + s) * d_size + d, sdpa/sdpa_utils.cuh:41); stats and the
// backward's workspace rows (stats2, delta) are fp32 [B, S_q].
#pragma once

#include <stdint.h>

namespace sdpa {

struct AttnShape {
    int B, S_q, S_kv, D_qk, D_v;
};

// Dropout and scaling constants derived once on the host.
struct AttnScalars {
    float scale;           // the op's `scale` attr
    float scale_log2;      // scale * log2(e): scores enter exp2 in this domain
    float keep_scale;      // 1 / (1 - p) when dropout is active, else 1
    uint32_t drop_threshold;  // element dropped iff (state >> 32) < drop_threshold
    int use_dropout;       // p > 1e-6 (sdpa/sdpa_fwd.cu.cc:136)
    int causal;            // top-left aligned: key j visible to query i iff j <= i
    uint64_t seed_offset;  // seed + offset (mod 2^64): the hash only sees the sum
};

struct FwdParams {
    const void* q;
    const void* k;
    const void* v;
    void* o;
    float* stats;
    AttnShape s;
    AttnScalars c;
};

struct BwdParams {
    const void* q;
    const void* k;
    const void* v;
    const void* o;
    const float* stats;
    const void* d_o;
    void* dq;
    void* dk;
    void* dv;
    // Workspace, written by the dQ kernel and read by the dK/dV kernel:
    float* stats2;  // [B, S_q]: stats_i * log2(e) + kGateShift (sdpa_device.h)
    float* delta;   // [B, S_q]: delta_i = sum_d dO[i,d] * O[i,d]
    AttnShape s;
    AttnScalars c;
};

}  // namespace sdpa
