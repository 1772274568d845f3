// sdpa_launch.h -- host-side launch helpers shared by the forward and backward
// launchers: compile-time dispatch over the padded feature widths and flags,
// and a launch wrapper that raises the dynamic-LDS limit once per kernel.
#pragma once

#include <hip/hip_runtime.h>

#include <mutex>
#include <type_traits>

#include "sdpa_params.h"

namespace sdpa {

enum class DType : int { F32 = 0, F16 = 1 };

// Padded feature width for D in [0, 128]: the MFMA tiles are 32 wide in the
// output direction, so every kernel is instantiated for 32, 64 and 128
// (the reference buckets max(D_qk, D_v) into 8/16/32/64/128,
// sdpa/sdpa_fwd.cu.cc:191-215; here D_qk and D_v are bucketed separately).
template <typename F>
hipError_t with_dim(int d, F&& f) {
    if (d <= 32) return f(std::integral_constant<int, 32>{});
    if (d <= 64) return f(std::integral_constant<int, 64>{});
    return f(std::integral_constant<int, 128>{});
}

template <typename F>
hipError_t with_bool(bool b, F&& f) {
    if (b) return f(std::true_type{});
    return f(std::false_type{});
}

// Launch `kern` with `lds` bytes of dynamic LDS.  The per-kernel attribute is
// set once per process (gfx950 has 160 KB of LDS per CU; kernels here use at
// most ~100 KB).
// The kernel is a template argument so that each kernel gets its own once-flag.
template <auto kern, typename... Args>
hipError_t launch_kernel(unsigned grid, unsigned block, size_t lds, hipStream_t stream,
                         const Args&... args) {
    static std::once_flag once;
    static hipError_t attr_err = hipSuccess;
    std::call_once(once, [&] {
        attr_err = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    });
    if (attr_err != hipSuccess) return attr_err;
    if (grid == 0) return hipSuccess;
    hipLaunchKernelGGL(kern, dim3(grid), dim3(block), lds, stream, args...);
    return hipGetLastError();
}

hipError_t launch_fwd(const FwdParams& p, DType dtype, bool vec, hipStream_t stream);
// phases: kBwdDq (dQ kernel, writes delta) and/or kBwdDkDv (reads delta).
constexpr int kBwdDq = 1, kBwdDkDv = 2;
hipError_t launch_bwd(const BwdParams& p, DType dtype, bool vec, int phases, hipStream_t stream);

// fp16 kernels fed by HBM -> LDS copies (sdpa_f16_fwd.hip, sdpa_f16_dq.hip,
// sdpa_f16_dkdv.hip).  They require D_qk and D_v to be multiples of 8 and
// every tensor 16-byte aligned.
hipError_t launch_fwd_f16_dma(const FwdParams& p, hipStream_t stream);
hipError_t launch_bwd_f16_dma(const BwdParams& p, int phases, hipStream_t stream);
// dQ phase of launch_bwd_f16_dma (sdpa_f16_dq.hip)
hipError_t launch_bwd_dq_f16_dma(const BwdParams& p, hipStream_t stream);
// dK/dV phase of launch_bwd_f16_dma at a 128-wide side (D_qk or D_v = 128;
// sdpa_f16_dkdv_split.hip); with p.ds set it also stores dS' (DsLayout)
hipError_t launch_bwd_dkdv_f16_split(const BwdParams& p, hipStream_t stream);

// dS path of the fp16 DMA backward (sdpa_f16_dq_ds.hip), for the shapes the
// split dK/dV kernels serve: the row values (stats2, delta), then
// launch_bwd_dkdv_f16_split with p.ds, then dQ from the stored dS'.
inline bool bwd_ds_shape(int D_qk, int D_v) { return D_qk > 64 || D_v > 64; }
hipError_t launch_bwd_rows_f16(const BwdParams& p, hipStream_t stream);
hipError_t launch_bwd_dq_ds_f16(const BwdParams& p, hipStream_t stream);
// The same path for fp32 (sdpa_f32_dq_ds.hip; its dK/dV phase is launch_bwd
// with p.ds set, which runs the fp32 split dK/dV kernel storing dS).
hipError_t launch_bwd_rows_f32(const BwdParams& p, hipStream_t stream);
hipError_t launch_bwd_dq_ds_f32(const BwdParams& p, hipStream_t stream);

}  // namespace sdpa
