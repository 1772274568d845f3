/*
 * sdpa_cpu.h -- C ABI of the host (CPU) kernels of the Sdpa / SdpaGrad ops,
 * the op's DEVICE_CPU registration.  They replace
 *     functor::FlashAttnFunctor<CPUDevice, T>       (sdpa/sdpa_cpu.cc:213-320)
 *     functor::FlashAttnGradFunctor<CPUDevice, T>   (sdpa/sdpa_cpu.cc:322-457)
 * behind the reference's DEVICE_CPU kernel registration
 * (sdpa/sdpa_cpu.cc:460-468).  libsdpa_cpu.so is product code for tensors
 * that live in host memory; it is never used for device tensors, and the GPU
 * library (sdpa_hip.h) does not call it.
 *
 * Conventions as in sdpa_hip.h: dense row-major [B,S,D] tensors, dtype
 * SDPA_CPU_DTYPE_F32 / SDPA_CPU_DTYPE_F16 (IEEE binary16), stats fp32
 * [B,S_q] in natural-log units, return value 0 or an sdpa_status_t code of
 * sdpa_hip.h (the argument checks are the same).  Pointers are host
 * pointers.  nthreads <= 0 uses every hardware thread.
 *
 * Semantics of the reference CPU functors: dropout is active iff p > 0
 * (sdpa_cpu.cc:232-235), p > 1 drops every element, p == 1 is rejected
 * (SDPA_ERR_DROPOUT_RANGE), the backward skips an element iff P < 1e-6
 * (sdpa_cpu.cc:384-385); products and accumulations run in fp32 (the
 * reference rounds half*half products and dK/dV to half, sdpa_cpu.cc:261,
 * 416-417; the results agree to within the fp16 tolerances).
 */
#ifndef SDPA_CPU_H_
#define SDPA_CPU_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SDPA_CPU_DTYPE_F32 0
#define SDPA_CPU_DTYPE_F16 1

/* Message for a status code (static storage, never NULL); the same codes and
 * messages as sdpa_hip_status_string, without the GPU library. */
const char* sdpa_cpu_status_string(int status);

/* The reference's argument checks of Sdpa / SdpaGrad, as sdpa_hip_check_fwd
 * and sdpa_hip_check_bwd (sdpa/sdpa_ops.cc:22-25,55-57,
 * sdpa/sdpa_cpu.cc:37-69,116-168): shapes as rank + dims, scalars rank 0;
 * the first failing check in the reference's order. */
int sdpa_cpu_check_fwd(int q_rank, const int64_t* q_shape, int k_rank, const int64_t* k_shape, int v_rank,
                       const int64_t* v_shape, int seed_rank, int offset_rank, int causal_mask);

int sdpa_cpu_check_bwd(int q_rank, const int64_t* q_shape, int k_rank, const int64_t* k_shape, int v_rank,
                       const int64_t* v_shape, int o_rank, const int64_t* o_shape, int stats_rank,
                       const int64_t* stats_shape, int do_rank, const int64_t* do_shape, int seed_rank,
                       int offset_rank, int causal_mask);

int sdpa_cpu_fwd(int dtype, const void* q, const void* k, const void* v, void* o, float* stats,
                 int B, int S_q, int S_kv, int D_qk, int D_v, float scale, float dropout,
                 int causal_mask, uint64_t seed, uint64_t offset, int nthreads);

int sdpa_cpu_bwd(int dtype, const void* q, const void* k, const void* v, const void* o,
                 const float* stats, const void* d_o, void* dq, void* dk, void* dv, int B, int S_q,
                 int S_kv, int D_qk, int D_v, float scale, float dropout, int causal_mask,
                 uint64_t seed, uint64_t offset, int nthreads);

#ifdef __cplusplus
}
#endif

#endif /* SDPA_CPU_H_ */
