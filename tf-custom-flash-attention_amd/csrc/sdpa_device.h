// sdpa_device.h -- device-side building blocks shared by the Sdpa / SdpaGrad
// kernels for gfx950 (CDNA4): MFMA wrappers, the dropout counter hash, LDS
// transpose reads and cross-lane reductions.
//
// MFMA lane layouts used throughout (64-lane wavefront, l = lane id,
// h = l / 32, verified on MI355X):
//   v_mfma_f32_32x32x16_f16  A: row l%32, k = 8h..8h+7      (8 halves)
//                            B: col l%32, k = 8h..8h+7      (8 halves)
//                            C: col l%32, row 8*(r/4) + 4h + r%4 for r = 0..15
//   v_mfma_f32_32x32x2_f32   A: row l%32, k = h; B: col l%32, k = h; C as above.
// An accumulator C[m][n] therefore holds column n in lane n%32 with the rows
// m spread inside the lane, which is exactly the B-operand layout of a
// following MFMA whose reduction runs over m -- provided the A operand lists
// the reduction index in the same (permuted) order.  Every kernel here uses
// that to chain GEMMs without an LDS round trip.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace sdpa {

typedef _Float16 half_t;
typedef half_t half8 __attribute__((ext_vector_type(8)));
typedef half_t half4 __attribute__((ext_vector_type(4)));
typedef half_t half2v __attribute__((ext_vector_type(2)));
typedef __fp16 fp16x4_tr __attribute__((vector_size(8)));  // operand type of the tr builtin
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx2 __attribute__((ext_vector_type(2)));

// Constants of the reference (sdpa/sdpa_utils.cuh:9-11).
constexpr float kEps = 1e-6f;
constexpr float kNegInf = -1e9f;
// 64-bit LCG step of the dropout hash (sdpa/sdpa_utils.cuh:13-19).
constexpr uint64_t kLcgMul = 6364136223846793005ULL;
constexpr uint64_t kLcgInc = 1442695040888963407ULL;

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
// The backward's P <= 1e-6 gate without a compare.  v_exp_f32 returns +0 for
// every argument below -126 (its results never go denormal, whatever the
// denormal mode), so P' = exp2(x - kGateShift) is 0 exactly when
// P = exp2(x) < 2^(kGateShift - 126) = 1e-6, and P = P' * kGateScale
// otherwise (kGateScale = 2^kGateShift).  The fp16 DMA backward kernels
// evaluate P' and fold kGateScale into factors they apply anyway.
constexpr float kGateShift = 106.068428f;   // 126 + log2(1e-6)
constexpr float kGateScale = 8.50703884e31f;  // 2^kGateShift
// Running-max sentinel in the log2 domain: finite, so exp2(x - m) never sees
// (-inf) - (-inf); masked scores are -inf and contribute exactly 0.
constexpr float kMaxSentinel = -1e30f;

__device__ __forceinline__ floatx16 mfma_f16(const half8& a, const half8& b, const floatx16& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ floatx16 mfma_f32(float a, float b, const floatx16& c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
// v_log_f32: log2, -inf at 0
__device__ __forceinline__ float fast_log2(float x) { return __builtin_amdgcn_logf(x); }

// Hi/lo split of P~ in the PV product.  A key sub-tile's P~ enters the fp16
// MFMA as one fp16 part, relative rounding 2^-11 per element; where a few
// keys carry a row's mass that moves o by up to 2^-11 |v|, which for |v| of
// a few units is more than half an fp16 ulp of o.  The kernels then add the
// remainder P~ - fp16(P~) as a second fp16 part (P~ to ~2^-22).  A sub-tile
// is split when some row of the wave has a score above the row's running
// log2-sum-exp (m + log2 l over the keys before it, refreshed once per key
// block) + kSplitLog2, i.e. one key of the sub-tile would hold more than 2^-3
// of the mass seen so far.  The log-sum-exp does not move when the running
// maximum is rescaled, and one refreshed less often is smaller, so the test
// only errs towards splitting.
constexpr float kSplitLog2 = -3.0f;

// Value of lane l^32 combined with the own value: permlane32_swap exchanges the
// upper half of the first operand with the lower half of the second, so the
// two outputs hold {own, partner} in some order for every lane.
__device__ __forceinline__ float xhalf_max(float x) {
    auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xhalf_sum(float x) {
    auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// ds_read_b64_tr_b16: inside each 16-lane group, lane j receives element e
// (e = 0..3) from the 64-bit row addressed by lane 4e + j/4 of the group, at
// 16-bit position j%4.  With lane i of the group pointing at
// X[row0 + i/4][col0 + 4*(i%4)], lane j receives X[row0 + e][col0 + j]:
// a 4 x 16 block of a row-major matrix arrives column-per-lane.
__device__ __forceinline__ half4 lds_read_tr(const half_t* p) {
    fp16x4_tr t = __builtin_amdgcn_ds_read_tr16_b64_v4f16(
        (__attribute__((address_space(3))) fp16x4_tr*)(p));
    return __builtin_bit_cast(half4, t);
}

__device__ __forceinline__ half2v cvt_pk(float a, float b) {
    half2v r;
    r[0] = (half_t)a;  // v_cvt_pk_f16_f32 (round to nearest even)
    r[1] = (half_t)b;
    return r;
}

// Dropout hash state for the element (b, i, j):
//   st(b,i,j) = (seed + offset + (b*S_q + i)*S_kv + j) * A + C   (mod 2^64)
// The element is dropped iff (float)(st >> 32) / 2^32 < p, which is
// equivalent to (st >> 32) < T(p) for the integer threshold computed on the
// host; st(b,i,j+n) = st(b,i,j) + n*A, so stepping along j is one 64-bit add.
__device__ __forceinline__ uint64_t lcg_state(uint64_t seed_offset, uint64_t row_index,
                                              uint64_t S_kv, uint64_t j) {
    return (seed_offset + row_index * S_kv + j) * kLcgMul + kLcgInc;
}
__device__ __forceinline__ bool lcg_keep(uint64_t state, uint32_t threshold) {
    return (uint32_t)(state >> 32) >= threshold;
}

// s_waitcnt vmcnt(0) after the operand rows a kernel loads into registers
// once, before its loop.  Without it the compiler's wait analysis, which
// merges the loop's entry state with its back edge, keeps those loads
// pending in every iteration and puts a vmcnt(0) before the loop's first use
// of them, which then also waits for every copy and store the iteration has
// in flight.
__device__ __forceinline__ void prologue_loads_landed() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// Wave-uniform "any lane" test.
__device__ __forceinline__ bool wave_any(bool p) { return __builtin_amdgcn_ballot_w64(p) != 0; }

}  // namespace sdpa
