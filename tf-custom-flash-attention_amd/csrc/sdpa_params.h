// sdpa_params.h -- kernel argument blocks shared by the host launchers and the
// HIP kernels.  Every tensor is dense row-major [B, S, D] (reference indexing
// (batch_offset + s) * d_size + d, sdpa/sdpa_utils.cuh:41); stats and the
// backward's workspace rows (stats2, delta) are fp32 [B, S_q].
#pragma once

#include <stdint.h>

#include <hip/hip_runtime.h>

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
    // Workspace, written by the dQ kernel (or the row kernel of the dS path)
    // and read by the dK/dV kernel:
    float* stats2;  // [B, S_q]: stats_i * log2(e) + kGateShift (sdpa_device.h)
    float* delta;   // [B, S_q]: delta_i = sum_d dO[i,d] * O[i,d]
    // dS path only (else null): dS' of every visited (key tile, query block),
    // written by the dK/dV kernel and read by the dQ kernel (DsLayout)
    void* ds;
    AttnShape s;
    AttnScalars c;
};

// Layout of the stored dS of the dS path.  The dK/dV kernel walks key tiles
// of 128 keys and query blocks of QBK queries (64 in the fp16 kernel, 32 in
// the fp32 one); under the causal mask key tile kt visits the query blocks
// qb >= qbb(kt) = min(128 kt, S_q) / QBK, else all of them.  Each visited
// (kt, qb) is a 16 KB chunk, and the chunks of a batch row follow each other
// kt-major, qb-minor.
//
// fp16 (DsLayout, QBK 64, dS' = dS (1-p)): inside a chunk, two 32-query
// sub-tiles t of 8 KB, each four 2 KB key groups (32 keys), each four
// 512-byte planes p of 32 slots of 16 bytes.  Slot slot(key, p) of plane
// p = 2 j + h holds the key's dS' at query positions 16 h + 8 j .. + 7: one
// store j of the dK/dV lane 32 h + key, so each store instruction writes 1 KB
// in whole 64-byte runs of four lanes.  The key order inside a plane
// (key ^ 4 p) puts the four planes' rows 0-3 in different LDS banks, for the
// dQ kernel's transposed read of the group copied as it lies.
//
// fp32 (DsLayout32, QBK 32, dS): inside a chunk, four 4 KB key groups (32
// keys), each four 1 KB quarters u, each two 512-byte halves h of 32 slots of
// 16 bytes.  Slot slot32(key, pos) of quarter u, half h holds the key's dS at
// query positions 16 h + 4 u .. + 3: store u of the dK/dV lane 32 h + key, so
// each store instruction writes 1 KB whole.  The key order inside a half
// (key ^ (u + 4 h)) puts the eight (u, h) slots of one key row in different
// LDS banks, for the dQ kernel's read of a key row by 32 lanes.
//
// In both, the 32 query positions of a sub-tile are in the order the dK/dV
// kernel's lanes hold them: position i is query 8 ((i >> 2) & 3) + 4 (i >> 4)
// + (i & 3) of the sub-tile.
template <int QBK_>
struct DsLayoutT {
    static constexpr int KT = 128, QBK = QBK_, R = KT / QBK, CHUNK = 16384;
    int S_q, QB, F, tiles;
    bool causal;
    __host__ __device__ DsLayoutT(int S_q_, int S_kv, bool causal_)
        : S_q(S_q_), QB((S_q_ + QBK - 1) / QBK), F(S_q_ / QBK), tiles((S_kv + KT - 1) / KT), causal(causal_) {}
    // first query block key tile kt visits
    __host__ __device__ int qbb(int kt) const { return !causal ? 0 : ((long long)KT * kt <= S_q ? R * kt : F); }
    // chunks of the key tiles before kt
    __host__ __device__ long long prefix(int kt) const {
        if (!causal) return (long long)kt * QB;
        const long long J = kt < S_q / KT + 1 ? kt : S_q / KT + 1;  // tiles j < kt with 128 j <= S_q
        return J * QB - R * (J * (J - 1) / 2) + (long long)(kt - J) * (QB - F);
    }
    __host__ __device__ long long per_row() const { return prefix(tiles); }
    // byte offset of chunk (b, kt, qb), qb >= qbb(kt)
    __host__ __device__ size_t offset(int b, int kt, int qb) const {
        return ((size_t)b * (size_t)per_row() + (size_t)prefix(kt) + (size_t)(qb - qbb(kt))) * CHUNK;
    }
    __host__ __device__ size_t bytes(int B) const { return (size_t)B * (size_t)per_row() * CHUNK; }
    // fp16: byte offset of (key, plane p) inside its 2 KB key group
    __host__ __device__ static constexpr int slot(int key, int p) { return p * 512 + (key ^ (4 * p)) * 16; }
    // fp32: byte offset of (key, query position) inside its 4 KB key group
    __host__ __device__ static constexpr int slot32(int key, int pos) {
        return 1024 * ((pos >> 2) & 3) + 512 * (pos >> 4) + 16 * (key ^ (((pos >> 2) & 3) + 4 * (pos >> 4))) +
               4 * (pos & 3);
    }
};
using DsLayout = DsLayoutT<64>;
using DsLayout32 = DsLayoutT<32>;

}  // namespace sdpa
