/*
 * sdpa_hip.h -- C ABI of the MI355X (gfx950) implementation of the Sdpa /
 * SdpaGrad TensorFlow custom ops of gravytrain777/tf-custom-flash-attention.
 *
 * This library replaces the reference's device seam
 *     functor::FlashAttnFunctor<GPUDevice, T>       (sdpa/sdpa.h:11-18)
 *     functor::FlashAttnGradFunctor<GPUDevice, T>   (sdpa/sdpa.h:20-34)
 * with plain-pointer entry points, plus the input validation the reference
 * performs in SdpaFwdOp::Compute / SdpaBwdOp::Compute (sdpa/sdpa_cpu.cc:29-87,
 * 105-192) so that every host binding reports the same errors.
 *
 * Conventions
 *   - Every tensor is dense row-major: q [B,S_q,D_qk], k [B,S_kv,D_qk],
 *     v [B,S_kv,D_v], o / do [B,S_q,D_v], stats [B,S_q] (fp32, natural log).
 *   - dtype: SDPA_DTYPE_F32 (float) or SDPA_DTYPE_F16 (IEEE binary16).
 *   - Pointers are device pointers; the caller owns every buffer (the
 *     library allocates nothing and keeps no per-call state).
 *   - Launches are asynchronous on `stream`; nothing synchronises.
 *   - Return value: SDPA_OK or an sdpa_status_t; sdpa_hip_status_string()
 *     gives the message (argument errors use the reference's wording).
 */
#ifndef SDPA_HIP_H_
#define SDPA_HIP_H_

#include <stddef.h>
#include <stdint.h>

/* The stream handle type of the HIP runtime (hip/hip_runtime_api.h declares
 * the same typedef), so that a host binding written in plain C or C++ needs
 * neither the HIP headers nor a HIP platform macro to include this file. */
typedef struct ihipStream_t* hipStream_t;

#ifdef __cplusplus
extern "C" {
#endif

#define SDPA_HIP_ABI_VERSION 1

typedef enum {
    SDPA_DTYPE_F32 = 0,
    SDPA_DTYPE_F16 = 1
} sdpa_dtype_t;

typedef enum {
    SDPA_OK = 0,
    /* argument errors, reference OP_REQUIRES order (sdpa/sdpa_cpu.cc:37-69, 116-168) */
    SDPA_ERR_SEED_NOT_SCALAR = 1,
    SDPA_ERR_OFFSET_NOT_SCALAR = 2,
    SDPA_ERR_K_BATCH = 3,
    SDPA_ERR_K_FEATURE = 4,
    SDPA_ERR_V_BATCH = 5,
    SDPA_ERR_V_SEQ = 6,
    SDPA_ERR_O_BATCH = 7,
    SDPA_ERR_O_SEQ = 8,
    SDPA_ERR_O_FEATURE = 9,
    SDPA_ERR_DO_BATCH = 10,
    SDPA_ERR_DO_SEQ = 11,
    SDPA_ERR_DO_FEATURE = 12,
    SDPA_ERR_S_BATCH = 13,
    SDPA_ERR_S_SEQ = 14,
    SDPA_ERR_CAUSAL_SEQ = 15,
    SDPA_ERR_FEATURE_TOO_LARGE = 16,
    /* shape-function error (sdpa/sdpa_ops.cc:22-25, 55-57) */
    SDPA_ERR_RANK = 17,
    /* errors of this library's own ABI */
    SDPA_ERR_DTYPE = 18,
    SDPA_ERR_NEGATIVE_DIM = 19,
    SDPA_ERR_NULL_POINTER = 20,
    SDPA_ERR_DROPOUT_RANGE = 21,
    SDPA_ERR_WORKSPACE = 22,
    SDPA_ERR_HIP = 23,
    SDPA_ERR_SCRATCH_LIMIT = 24,
    SDPA_ERR_DS_PATH = 25
} sdpa_status_t;

/* Message for a status code (static storage, never NULL). */
const char* sdpa_hip_status_string(int status);

/* HIP error of the most recent SDPA_ERR_HIP returned on this thread. */
int sdpa_hip_last_hip_error(void);

/* ---- validation (host only, no device work) -------------------------------
 * Mirrors SdpaFwdOp::Compute (sdpa/sdpa_cpu.cc:37-69) plus the Sdpa shape fn
 * (sdpa/sdpa_ops.cc:22-25): shapes are given as rank + dims; a scalar has
 * rank 0.  Returns the first failing check in the reference's order.       */
int sdpa_hip_check_fwd(int q_rank, const int64_t* q_shape, int k_rank, const int64_t* k_shape,
                       int v_rank, const int64_t* v_shape, int seed_rank, int offset_rank,
                       int causal_mask);

/* Mirrors SdpaBwdOp::Compute (sdpa/sdpa_cpu.cc:116-168) and the SdpaGrad
 * shape fn (sdpa/sdpa_ops.cc:55-57).                                        */
int sdpa_hip_check_bwd(int q_rank, const int64_t* q_shape, int k_rank, const int64_t* k_shape,
                       int v_rank, const int64_t* v_shape, int o_rank, const int64_t* o_shape,
                       int stats_rank, const int64_t* stats_shape, int do_rank,
                       const int64_t* do_shape, int seed_rank, int offset_rank, int causal_mask);

/* ---- forward: replaces FlashAttnFunctor<GPUDevice,T> (sdpa/sdpa_fwd.cu.cc:176-240)
 * o     = softmax(scale * q k^T [causal]) (dropout) v     [B,S_q,D_v], dtype
 * stats = m + log(l + 1e-6)                               [B,S_q] fp32
 * Requires max(D_qk, D_v) <= 128 and, with causal_mask, S_q == S_kv.
 * dropout <= 1e-6 disables dropout (as the reference GPU); dropout > 1 drops
 * every element as the reference does (o = 0, the usual stats; in the
 * backward dV = 0 and dS = -P delta); dropout == 1 returns
 * SDPA_ERR_DROPOUT_RANGE (the reference would scale by 1 / 0).  */
int sdpa_hip_fwd(int dtype, const void* q, const void* k, const void* v, void* o, float* stats,
                 int B, int S_q, int S_kv, int D_qk, int D_v, float scale, float dropout,
                 int causal_mask, uint64_t seed, uint64_t offset, hipStream_t stream);

/* ---- backward: replaces FlashAttnGradFunctor<GPUDevice,T> (sdpa/sdpa_bwd.cu.cc:347-453)
 * Needs a device workspace of sdpa_hip_bwd_workspace_bytes(B, S_q) bytes
 * (two fp32 values per query row: stats * log2(e) and delta = sum_d dO * O),
 * provided by the caller as the TF op does with allocate_temp.              */
size_t sdpa_hip_bwd_workspace_bytes(int B, int S_q);

int sdpa_hip_bwd(int dtype, const void* q, const void* k, const void* v, const void* o,
                 const float* stats, const void* d_o, void* dq, void* dk, void* dv,
                 void* workspace, size_t workspace_bytes, int B, int S_q, int S_kv, int D_qk,
                 int D_v, float scale, float dropout, int causal_mask, uint64_t seed,
                 uint64_t offset, hipStream_t stream);

/* The two launches of sdpa_hip_bwd as separate calls, same arguments, same
 * stream order required (the reference launches its two backward kernels
 * back to back, sdpa/sdpa_bwd.cu.cc:402-405):
 *   sdpa_hip_bwd_dq   -- dQ, and the per-row values into the workspace;
 *   sdpa_hip_bwd_dkdv -- dK and dV, reading the values left in the workspace
 *                        by a preceding sdpa_hip_bwd_dq with the same inputs.
 * sdpa_hip_bwd == sdpa_hip_bwd_dq followed by sdpa_hip_bwd_dkdv.            */
int sdpa_hip_bwd_dq(int dtype, const void* q, const void* k, const void* v, const void* o,
                    const float* stats, const void* d_o, void* dq, void* workspace,
                    size_t workspace_bytes, int B, int S_q, int S_kv, int D_qk, int D_v,
                    float scale, float dropout, int causal_mask, uint64_t seed, uint64_t offset,
                    hipStream_t stream);

int sdpa_hip_bwd_dkdv(int dtype, const void* q, const void* k, const void* v, const float* stats,
                      const void* d_o, void* dk, void* dv, const void* workspace,
                      size_t workspace_bytes, int B, int S_q, int S_kv, int D_qk, int D_v,
                      float scale, float dropout, int causal_mask, uint64_t seed,
                      uint64_t offset, hipStream_t stream);

/* ---- backward, dS path --------------------------------------------------
 * No counterpart in the reference (an MI355X choice of how its two backward
 * kernels divide the work).  For float16 and float32 with a feature size
 * over 64, the dK/dV kernel can store the dS it forms (in T, every visited
 * score: about B * S_q * S_kv * sizeof(T) / 2 bytes under the causal mask,
 * twice that without) and dQ is then one product with it, instead of a
 * kernel that forms S, P, dP and dS again.  sdpa_hip_bwd takes this path whenever the shape qualifies, the
 * tensors are 16-byte aligned and workspace_bytes is at least
 * sdpa_hip_bwd_workspace_bytes_ds(...); with a smaller workspace (at least
 * sdpa_hip_bwd_workspace_bytes(B, S_q)) it takes the other one.  For shapes
 * that do not qualify the function returns sdpa_hip_bwd_workspace_bytes. */
size_t sdpa_hip_bwd_workspace_bytes_ds(int dtype, int B, int S_q, int S_kv, int D_qk, int D_v,
                                       int causal_mask);

/* The three launches of the dS path as separate calls (same arguments as
 * sdpa_hip_bwd; each phase reads what the previous one left in the workspace,
 * in stream order):
 *   phase 0 -- the per-row values (stats * log2(e), delta) into the workspace;
 *   phase 1 -- dK, dV and the stored dS;
 *   phase 2 -- dQ from the stored dS.
 * Returns SDPA_ERR_DS_PATH where sdpa_hip_bwd would not take the dS path.  */
int sdpa_hip_bwd_ds_phase(int phase, int dtype, const void* q, const void* k, const void* v,
                          const void* o, const float* stats, const void* d_o, void* dq, void* dk,
                          void* dv, void* workspace, size_t workspace_bytes, int B, int S_q,
                          int S_kv, int D_qk, int D_v, float scale, float dropout, int causal_mask,
                          uint64_t seed, uint64_t offset, hipStream_t stream);

/* ---- backward that allocates nothing ---------------------------------------
 * No counterpart in the reference.  For callers that cannot allocate device
 * memory or pass a workspace: code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc.  Same arguments and results as
 * sdpa_hip_bwd without the workspace: the per-query-row values live in a
 * static device array of SDPA_HIP_NOALLOC_SCRATCH_BYTES per GPU (8 bytes per
 * query row, so B * S_q <= 2,097,152; larger problems return
 * SDPA_ERR_SCRATCH_LIMIT).  Calls no hipMalloc / hipFree; its first call on
 * a device looks up that device's copy of the array (hipGetSymbolAddress).
 * Every call on one GPU shares that GPU's array: calls that overlap on one
 * GPU (different streams, or host threads without ordering) race.          */
#define SDPA_HIP_NOALLOC_SCRATCH_BYTES (16u << 20)

int sdpa_hip_bwd_noalloc(int dtype, const void* q, const void* k, const void* v, const void* o,
                         const float* stats, const void* d_o, void* dq, void* dk, void* dv, int B,
                         int S_q, int S_kv, int D_qk, int D_v, float scale, float dropout,
                         int causal_mask, uint64_t seed, uint64_t offset, hipStream_t stream);

/* ---- dropout hash (sdpa/sdpa_utils.cuh:13-19, sdpa/sdpa_cpu.cc:198-211) ----
 * Integer form of the reference's predicate (float)(st >> 32) / 2^32 < p:
 * element dropped iff (st >> 32) < T(p).  Returns T(p) as a 64-bit value
 * (2^32 means "every element dropped"; only reachable for p > 1).           */
uint64_t sdpa_hip_drop_threshold(float dropout);

/* Device dump of the keep mask the kernels apply (1 = kept), uint8
 * [B, S_q, S_kv], computed by the kernels' own hash code.  For tests.       */
int sdpa_hip_dropout_mask(uint8_t* keep, int B, int S_q, int S_kv, float dropout, uint64_t seed,
                          uint64_t offset, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* SDPA_HIP_H_ */
