// sdpa_capi.hip -- the extern "C" entry points declared in include/sdpa_hip.h:
// argument validation with the reference's messages, the dropout threshold,
// and dispatch to the forward / backward launchers.
#include <math.h>
#include <stdint.h>

#include <mutex>

#include "sdpa_hip.h"
#include "sdpa_checks.h"
#include "sdpa_device.h"
#include "sdpa_launch.h"
#include "sdpa_params.h"

namespace {

thread_local int g_last_hip_error = 0;

int hip_status(hipError_t e) {
    if (e == hipSuccess) return SDPA_OK;
    g_last_hip_error = (int)e;
    return SDPA_ERR_HIP;
}

bool aligned16(const void* ptr) { return ((uintptr_t)ptr & 15u) == 0; }

// Smallest uint32 value v with (float)v / 2^32 >= p, as a 64-bit number
// (2^32 if none).  (float)v rounds to nearest even, which is monotone in v,
// so "u < p" is the prefix v < T(p) of the 32-bit range.  T(p) is not
// floor(p * 2^32): e.g. T(0.1f) = 0x19999991, T(0.2f) = 0x33333321.
uint64_t drop_threshold_impl(float p) {
    if (!(p > 0.0f)) return 0;  // nothing satisfies u < p (also NaN)
    const float P = p * 4294967296.0f;  // exact: scaling by a power of two
    if (!((float)4294967295u >= P)) return 1ull << 32;
    uint64_t lo = 0, hi = 0xFFFFFFFFull;
    while (lo < hi) {
        const uint64_t mid = (lo + hi) >> 1;
        if ((float)(uint32_t)mid >= P) hi = mid;
        else lo = mid + 1;
    }
    return lo;
}

// Host-side derivation of the per-call constants (reference:
// dp_inverse = 1 / (1 - p) when p > EPSF, sdpa/sdpa_fwd.cu.cc:20).
// dropout > 1 drops every element in the reference (u <= 1 < p,
// sdpa/sdpa_fwd.cu.cc:136-146, sdpa/sdpa_bwd.cu.cc:135-157): o = 0 with the
// usual statistics (l sums the undropped probabilities), dV = 0 and
// dS = -P delta everywhere.  Here that is keep_scale = 0: the forward runs
// without dropout and scales o by 0; the backward runs with dropout, where
// every kernel forms dS = P (keep ? dP keep_scale - delta : -delta), i.e.
// -P delta for kept and dropped elements alike, and scales dV by keep_scale.
sdpa::AttnScalars make_scalars(float scale, float dropout, int causal, uint64_t seed, uint64_t offset,
                               bool backward) {
    sdpa::AttnScalars c{};
    c.scale = scale;
    c.scale_log2 = scale * sdpa::kLog2e;
    if (dropout > 1.0f) {
        c.use_dropout = backward ? 1 : 0;
        c.keep_scale = 0.0f;
        c.drop_threshold = 0xFFFFFFFFu;  // immaterial with keep_scale = 0
    } else {
        c.use_dropout = dropout > sdpa::kEps ? 1 : 0;
        c.keep_scale = c.use_dropout ? 1.0f / (1.0f - dropout) : 1.0f;
        c.drop_threshold = c.use_dropout ? (uint32_t)drop_threshold_impl(dropout) : 0u;
    }
    c.causal = causal ? 1 : 0;
    c.seed_offset = seed + offset;
    return c;
}

int check_common(int dtype, int B, int S_q, int S_kv, int D_qk, int D_v, float dropout, int causal) {
    if (dtype != SDPA_DTYPE_F32 && dtype != SDPA_DTYPE_F16) return SDPA_ERR_DTYPE;
    if (B < 0 || S_q < 0 || S_kv < 0 || D_qk < 0 || D_v < 0) return SDPA_ERR_NEGATIVE_DIM;
    if (causal && S_q != S_kv) return SDPA_ERR_CAUSAL_SEQ;
    if ((D_qk > D_v ? D_qk : D_v) > 128) return SDPA_ERR_FEATURE_TOO_LARGE;
    if (dropout == 1.0f) return SDPA_ERR_DROPOUT_RANGE;  // the reference divides by 1 - p
    return SDPA_OK;
}

bool vec_ok(int dtype, int D_qk, int D_v, std::initializer_list<const void*> ptrs) {
    const int w = dtype == SDPA_DTYPE_F16 ? 8 : 4;  // elements per 16-byte chunk
    if (D_qk % w != 0 || D_v % w != 0) return false;
    for (const void* p : ptrs)
        if (!aligned16(p)) return false;
    return true;
}

// keep[b, i, j] from the same hash code the attention kernels use.
// use_dropout: 0 keeps every element, 1 applies the hash test, 2 drops every
// element (dropout > 1).
__global__ void dropout_mask_kernel(uint8_t* keep, int B, int S_q, int S_kv, int use_dropout,
                                    uint32_t thr, uint64_t seed_offset) {
    const uint64_t total = (uint64_t)B * S_q * S_kv;
    for (uint64_t idx = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += (uint64_t)gridDim.x * blockDim.x) {
        const uint64_t row = idx / (uint64_t)S_kv, j = idx % (uint64_t)S_kv;
        keep[idx] = use_dropout == 2 ? 0
                    : use_dropout ? (uint8_t)sdpa::lcg_keep(sdpa::lcg_state(seed_offset, row, S_kv, j), thr)
                                  : 1;
    }
}

}  // namespace

extern "C" {

const char* sdpa_hip_status_string(int status) { return sdpa::status_message(status); }

int sdpa_hip_last_hip_error(void) { return g_last_hip_error; }

int sdpa_hip_check_fwd(int q_rank, const int64_t* q, int k_rank, const int64_t* k, int v_rank,
                       const int64_t* v, int seed_rank, int offset_rank, int causal_mask) {
    return sdpa::check_fwd_shapes(q_rank, q, k_rank, k, v_rank, v, seed_rank, offset_rank, causal_mask);
}

int sdpa_hip_check_bwd(int q_rank, const int64_t* q, int k_rank, const int64_t* k, int v_rank,
                       const int64_t* v, int o_rank, const int64_t* o, int stats_rank,
                       const int64_t* st, int do_rank, const int64_t* d_o, int seed_rank,
                       int offset_rank, int causal_mask) {
    return sdpa::check_bwd_shapes(q_rank, q, k_rank, k, v_rank, v, o_rank, o, stats_rank, st, do_rank, d_o,
                                  seed_rank, offset_rank, causal_mask);
}

int sdpa_hip_fwd(int dtype, const void* q, const void* k, const void* v, void* o, float* stats,
                 int B, int S_q, int S_kv, int D_qk, int D_v, float scale, float dropout,
                 int causal_mask, uint64_t seed, uint64_t offset, hipStream_t stream) {
    int st = check_common(dtype, B, S_q, S_kv, D_qk, D_v, dropout, causal_mask);
    if (st != SDPA_OK) return st;
    if ((size_t)B * S_q == 0) return SDPA_OK;  // empty grid: nothing to do
    if (!stats || (D_v > 0 && !o) || (D_qk > 0 && (!q || (S_kv > 0 && !k))) || (S_kv > 0 && D_v > 0 && !v))
        return SDPA_ERR_NULL_POINTER;
    sdpa::FwdParams p{};
    p.q = q;
    p.k = k;
    p.v = v;
    p.o = o;
    p.stats = stats;
    p.s = sdpa::AttnShape{B, S_q, S_kv, D_qk, D_v};
    p.c = make_scalars(scale, dropout, causal_mask, seed, offset, false);
    const bool vec = vec_ok(dtype, D_qk, D_v, {q, k, v, o});
    if (dtype == SDPA_DTYPE_F16 && vec) return hip_status(sdpa::launch_fwd_f16_dma(p, stream));
    return hip_status(sdpa::launch_fwd(p, (sdpa::DType)dtype, vec, stream));
}

size_t sdpa_hip_bwd_workspace_bytes(int B, int S_q) {
    if (B <= 0 || S_q <= 0) return 0;
    // stats * log2(e) and delta, one fp32 row each per query row.
    const size_t bytes = 2 * (size_t)B * (size_t)S_q * sizeof(float);
    return (bytes + 255) & ~(size_t)255;
}

}  // extern "C"

namespace {
// The dS path's shapes: fp16 or fp32 through a split dK/dV kernel, nothing
// empty.
bool ds_shape(int dtype, int B, int S_q, int S_kv, int D_qk, int D_v) {
    return (dtype == SDPA_DTYPE_F16 || dtype == SDPA_DTYPE_F32) && B > 0 && S_q > 0 && S_kv > 0 && D_qk > 0 &&
           D_v > 0 && sdpa::bwd_ds_shape(D_qk, D_v);
}
}  // namespace

extern "C" {

size_t sdpa_hip_bwd_workspace_bytes_ds(int dtype, int B, int S_q, int S_kv, int D_qk, int D_v,
                                       int causal_mask) {
    const size_t rows = sdpa_hip_bwd_workspace_bytes(B, S_q);
    if (!ds_shape(dtype, B, S_q, S_kv, D_qk, D_v) || D_qk > 128 || D_v > 128) return rows;
    // the row values first (a multiple of 256 bytes), the stored dS after them
    if (dtype == SDPA_DTYPE_F32) return rows + sdpa::DsLayout32(S_q, S_kv, causal_mask != 0).bytes(B);
    return rows + sdpa::DsLayout(S_q, S_kv, causal_mask != 0).bytes(B);
}

}  // extern "C"

namespace {
// Which launches a backward entry point makes:
//   kRecompute -- `phases` of the path that forms dS in both kernels (dQ
//                 first, it leaves the row values; then dK/dV);
//   kAuto      -- all of it, by the dS path when the workspace allows;
//   kDs0..2    -- one phase of the dS path (rows, dK/dV + dS, dQ).
enum Mode { kRecompute, kAuto, kDs0, kDs1, kDs2 };

// Shared body of the backward entry points.
int bwd_entry(Mode mode, int phases, int dtype, const void* q, const void* k, const void* v,
              const void* o, const float* stats, const void* d_o, void* dq, void* dk, void* dv,
              void* workspace, size_t workspace_bytes, int B, int S_q, int S_kv, int D_qk, int D_v,
              float scale, float dropout, int causal_mask, uint64_t seed, uint64_t offset,
              hipStream_t stream) {
    int st = check_common(dtype, B, S_q, S_kv, D_qk, D_v, dropout, causal_mask);
    if (st != SDPA_OK) return st;
    const bool ds_phase = mode == kDs0 || mode == kDs1 || mode == kDs2;
    if (B == 0) return SDPA_OK;
    const size_t rows_bytes = sdpa_hip_bwd_workspace_bytes(B, S_q);
    if (workspace_bytes < rows_bytes) return SDPA_ERR_WORKSPACE;
    const bool has_q = (size_t)S_q > 0, has_kv = (size_t)S_kv > 0;
    // what the call computes (every launch of the dS path needs the rows of
    // phase 0, so the full call checks all of its inputs)
    const bool want_dq = ds_phase ? mode == kDs2 : (mode == kAuto || (phases & sdpa::kBwdDq));
    const bool want_kv = ds_phase ? mode == kDs1 : (mode == kAuto || (phases & sdpa::kBwdDkDv));
    const bool want_rows = ds_phase ? mode == kDs0 : want_dq;
    if ((has_q && !workspace) || (has_q && !ds_phase && !stats) || (want_rows && has_q && !stats) ||
        (has_q && D_qk > 0 && !q && (want_kv || !ds_phase)) ||
        (has_q && D_v > 0 && !d_o && (want_kv || want_rows)) ||
        (want_dq && has_q && D_qk > 0 && !dq) || (want_rows && has_q && D_v > 0 && !o) ||
        (has_kv && D_qk > 0 && !k && (want_kv || want_dq)) || (has_kv && D_v > 0 && !v && (want_kv || !ds_phase)) ||
        (want_kv && has_kv && D_qk > 0 && !dk) || (want_kv && has_kv && D_v > 0 && !dv))
        return SDPA_ERR_NULL_POINTER;
    sdpa::BwdParams p{};
    p.q = q;
    p.k = k;
    p.v = v;
    p.o = o;
    p.stats = stats;
    p.d_o = d_o;
    p.dq = dq;
    p.dk = dk;
    p.dv = dv;
    p.stats2 = static_cast<float*>(workspace);
    p.delta = static_cast<float*>(workspace) + (size_t)B * S_q;
    p.ds = nullptr;
    p.s = sdpa::AttnShape{B, S_q, S_kv, D_qk, D_v};
    p.c = make_scalars(scale, dropout, causal_mask, seed, offset, true);
    const bool vec = vec_ok(dtype, D_qk, D_v,
                            {q, k, v, d_o, want_rows ? o : nullptr, want_dq ? dq : nullptr,
                             want_kv ? dk : nullptr, want_kv ? dv : nullptr});
    // the dS path: its shapes, aligned tensors, and the workspace for dS
    const bool ds_ok = vec && ds_shape(dtype, B, S_q, S_kv, D_qk, D_v) &&
                       workspace_bytes >= sdpa_hip_bwd_workspace_bytes_ds(dtype, B, S_q, S_kv, D_qk, D_v,
                                                                          causal_mask);
    if (ds_phase && !ds_ok) return SDPA_ERR_DS_PATH;
    if (ds_phase || (mode == kAuto && ds_ok)) {
        p.ds = static_cast<unsigned char*>(workspace) + rows_bytes;
        hipError_t e = hipSuccess;
        const bool f16 = dtype == SDPA_DTYPE_F16;
        if (mode == kAuto || mode == kDs0)
            e = f16 ? sdpa::launch_bwd_rows_f16(p, stream) : sdpa::launch_bwd_rows_f32(p, stream);
        if (e == hipSuccess && (mode == kAuto || mode == kDs1))
            e = f16 ? sdpa::launch_bwd_dkdv_f16_split(p, stream)
                    : sdpa::launch_bwd(p, sdpa::DType::F32, true, sdpa::kBwdDkDv, stream);
        if (e == hipSuccess && (mode == kAuto || mode == kDs2))
            e = f16 ? sdpa::launch_bwd_dq_ds_f16(p, stream) : sdpa::launch_bwd_dq_ds_f32(p, stream);
        return hip_status(e);
    }
    const int ph = mode == kAuto ? (sdpa::kBwdDq | sdpa::kBwdDkDv) : phases;
    if (dtype == SDPA_DTYPE_F16 && vec) return hip_status(sdpa::launch_bwd_f16_dma(p, ph, stream));
    return hip_status(sdpa::launch_bwd(p, (sdpa::DType)dtype, vec, ph, stream));
}
}  // namespace

extern "C" {

int sdpa_hip_bwd(int dtype, const void* q, const void* k, const void* v, const void* o,
                 const float* stats, const void* d_o, void* dq, void* dk, void* dv,
                 void* workspace, size_t workspace_bytes, int B, int S_q, int S_kv, int D_qk,
                 int D_v, float scale, float dropout, int causal_mask, uint64_t seed,
                 uint64_t offset, hipStream_t stream) {
    return bwd_entry(kAuto, 0, dtype, q, k, v, o, stats, d_o, dq, dk, dv, workspace, workspace_bytes, B,
                     S_q, S_kv, D_qk, D_v, scale, dropout, causal_mask, seed, offset, stream);
}

int sdpa_hip_bwd_dq(int dtype, const void* q, const void* k, const void* v, const void* o,
                    const float* stats, const void* d_o, void* dq, void* workspace,
                    size_t workspace_bytes, int B, int S_q, int S_kv, int D_qk, int D_v,
                    float scale, float dropout, int causal_mask, uint64_t seed, uint64_t offset,
                    hipStream_t stream) {
    return bwd_entry(kRecompute, sdpa::kBwdDq, dtype, q, k, v, o, stats, d_o, dq, nullptr, nullptr,
                     workspace, workspace_bytes, B, S_q, S_kv, D_qk, D_v, scale, dropout, causal_mask,
                     seed, offset, stream);
}

int sdpa_hip_bwd_dkdv(int dtype, const void* q, const void* k, const void* v, const float* stats,
                      const void* d_o, void* dk, void* dv, const void* workspace,
                      size_t workspace_bytes, int B, int S_q, int S_kv, int D_qk, int D_v,
                      float scale, float dropout, int causal_mask, uint64_t seed,
                      uint64_t offset, hipStream_t stream) {
    return bwd_entry(kRecompute, sdpa::kBwdDkDv, dtype, q, k, v, nullptr, stats, d_o, nullptr, dk, dv,
                     const_cast<void*>(workspace), workspace_bytes, B, S_q, S_kv, D_qk, D_v, scale,
                     dropout, causal_mask, seed, offset, stream);
}

int sdpa_hip_bwd_ds_phase(int phase, int dtype, const void* q, const void* k, const void* v,
                          const void* o, const float* stats, const void* d_o, void* dq, void* dk,
                          void* dv, void* workspace, size_t workspace_bytes, int B, int S_q,
                          int S_kv, int D_qk, int D_v, float scale, float dropout, int causal_mask,
                          uint64_t seed, uint64_t offset, hipStream_t stream) {
    if (phase < 0 || phase > 2) return SDPA_ERR_DS_PATH;
    const Mode m = phase == 0 ? kDs0 : (phase == 1 ? kDs1 : kDs2);
    return bwd_entry(m, 0, dtype, q, k, v, o, stats, d_o, dq, dk, dv, workspace, workspace_bytes, B, S_q,
                     S_kv, D_qk, D_v, scale, dropout, causal_mask, seed, offset, stream);
}

}  // extern "C"

// ---------------------------------------------------------------------------
// Static scratch of sdpa_hip_bwd_noalloc: the backward's per-query-row
// workspace (stats2, delta) for callers that cannot allocate.  Each device the
// library runs on holds its own copy from module load until the process ends.
// Host code never uses the array's name as an address (on the host it is a
// stand-in, not device memory): the device address comes from
// hipGetSymbolAddress, once per device, with that device current.
// ---------------------------------------------------------------------------
static __device__ __align__(256) unsigned char scratch[SDPA_HIP_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices];  // device address of `scratch` per device id

int scratch_on_current_device(void** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_status(e);
    if (dev < 0 || dev >= kMaxDevices) return hip_status(hipErrorInvalidDevice);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_ptr[dev] == nullptr) {
        void* ptr = nullptr;
        e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return hip_status(e);
        if (ptr == nullptr) return hip_status(hipErrorInvalidSymbol);
        g_scratch_ptr[dev] = ptr;
    }
    *out = g_scratch_ptr[dev];
    return SDPA_OK;
}
}  // namespace

extern "C" {

int sdpa_hip_bwd_noalloc(int dtype, const void* q, const void* k, const void* v, const void* o,
                         const float* stats, const void* d_o, void* dq, void* dk, void* dv, int B,
                         int S_q, int S_kv, int D_qk, int D_v, float scale, float dropout,
                         int causal_mask, uint64_t seed, uint64_t offset, hipStream_t stream) {
    int st = check_common(dtype, B, S_q, S_kv, D_qk, D_v, dropout, causal_mask);
    if (st != SDPA_OK) return st;
    const size_t need = sdpa_hip_bwd_workspace_bytes(B, S_q);
    if (need > (size_t)SDPA_HIP_NOALLOC_SCRATCH_BYTES) return SDPA_ERR_SCRATCH_LIMIT;
    void* ws = nullptr;
    if (need > 0) {
        st = scratch_on_current_device(&ws);
        if (st != SDPA_OK) return st;
    }
    // The kernels write every workspace row before reading it (dQ kernel,
    // then dK/dV kernel on the same stream): nothing needs clearing.
    return bwd_entry(kRecompute, sdpa::kBwdDq | sdpa::kBwdDkDv, dtype, q, k, v, o, stats, d_o, dq, dk, dv, ws,
                     need, B, S_q, S_kv, D_qk, D_v, scale, dropout, causal_mask, seed, offset,
                     stream);
}

uint64_t sdpa_hip_drop_threshold(float dropout) { return drop_threshold_impl(dropout); }

int sdpa_hip_dropout_mask(uint8_t* keep, int B, int S_q, int S_kv, float dropout, uint64_t seed,
                          uint64_t offset, hipStream_t stream) {
    if (B < 0 || S_q < 0 || S_kv < 0) return SDPA_ERR_NEGATIVE_DIM;
    if (dropout == 1.0f) return SDPA_ERR_DROPOUT_RANGE;
    const uint64_t total = (uint64_t)B * S_q * S_kv;
    if (total == 0) return SDPA_OK;
    if (!keep) return SDPA_ERR_NULL_POINTER;
    const sdpa::AttnScalars c = make_scalars(1.0f, dropout, 0, seed, offset, false);
    const uint64_t blocks = (total + 255) / 256;
    const unsigned grid = (unsigned)(blocks < 65536 ? blocks : 65536);
    // dropout > 1: every element dropped (use_dropout with an all-dropping test)
    const bool all = dropout > 1.0f;
    hipLaunchKernelGGL(dropout_mask_kernel, dim3(grid), dim3(256), 0, stream, keep, B, S_q, S_kv,
                       all ? 2 : c.use_dropout, c.drop_threshold, c.seed_offset);
    return hip_status(hipGetLastError());
}

}  // extern "C"
