// sdpa_kernels.cc -- TensorFlow OpKernels of Sdpa / SdpaGrad for the MI355X
// build, registered for DEVICE_GPU (the HIP kernels of libsdpa_hip.so,
// include/sdpa_hip.h) and DEVICE_CPU (the host kernels of libsdpa_cpu.so,
// include/sdpa_cpu.h), for T in {float, half}, with seed and offset in host
// memory on the GPU -- the registrations of sdpa/sdpa_cpu.cc:460-488.
//
// Compute follows SdpaFwdOp / SdpaBwdOp (sdpa/sdpa_cpu.cc:29-87, 105-192):
// attributes read once at construction (the kernels keep no other state and
// are re-entrant), input checks with the reference's messages, outputs
// allocated by TensorFlow, then one call into the device's C ABI.  The checks
// are the C ABI's (sdpa_hip_check_fwd / _bwd), which run the reference's
// OP_REQUIRES sequence in its order.  GPU launches go to the op's compute
// stream and are asynchronous; a launch failure becomes errors::Internal
// where the reference aborts via TF_CHECK_OK.
#define EIGEN_USE_THREADS
#define EIGEN_USE_GPU

#include <algorithm>
#include <cstdint>

#include "tensorflow/core/framework/op_kernel.h"
#include "tensorflow/core/framework/register_types.h"
#include "sdpa_cpu.h"
#include "sdpa_hip.h"

namespace tensorflow {

using CPUDevice = Eigen::ThreadPoolDevice;
using GPUDevice = Eigen::GpuDevice;

namespace {

template <typename T>
constexpr int dtype_code() {
    return std::is_same<T, Eigen::half>::value ? SDPA_DTYPE_F16 : SDPA_DTYPE_F32;
}

Status FromSdpa(int rc) {
    if (rc == SDPA_OK) return OkStatus();
    if (rc == SDPA_ERR_HIP)
        return errors::Internal(sdpa_hip_status_string(rc), " (hip error ", sdpa_hip_last_hip_error(), ")");
    return errors::InvalidArgument(sdpa_hip_status_string(rc));
}

// Rank and leading dimensions of a tensor, as the C ABI checks take them.
struct Dims {
    int rank;
    int64_t d[3];
    explicit Dims(const Tensor& t) : rank(t.dims()), d{0, 0, 0} {
        for (int i = 0; i < rank && i < 3; ++i) d[i] = t.dim_size(i);
    }
};

// The per-device half of Compute: one call into that device's C ABI.
template <typename Device>
struct Backend;

template <>
struct Backend<CPUDevice> {
    static int threads(OpKernelContext* ctx) {
        return ctx->device()->tensorflow_cpu_worker_threads()->num_threads;
    }
    static Status fwd(OpKernelContext* ctx, int dt, const void* q, const void* k, const void* v, void* o,
                      float* stats, int B, int S_q, int S_kv, int D_qk, int D_v, float scale, float dropout,
                      bool causal, uint64 seed, uint64 offset) {
        return FromSdpa(sdpa_cpu_fwd(dt, q, k, v, o, stats, B, S_q, S_kv, D_qk, D_v, scale, dropout, causal,
                                     seed, offset, threads(ctx)));
    }
    static Status bwd(OpKernelContext* ctx, int dt, const void* q, const void* k, const void* v, const void* o,
                      const float* stats, const void* d_o, void* dq, void* dk, void* dv, int B, int S_q,
                      int S_kv, int D_qk, int D_v, float scale, float dropout, bool causal, uint64 seed,
                      uint64 offset) {
        return FromSdpa(sdpa_cpu_bwd(dt, q, k, v, o, stats, d_o, dq, dk, dv, B, S_q, S_kv, D_qk, D_v, scale,
                                     dropout, causal, seed, offset, threads(ctx)));
    }
};

template <>
struct Backend<GPUDevice> {
    static hipStream_t stream(OpKernelContext* ctx) {
        return reinterpret_cast<hipStream_t>(ctx->eigen_device<GPUDevice>().stream());
    }
    static Status fwd(OpKernelContext* ctx, int dt, const void* q, const void* k, const void* v, void* o,
                      float* stats, int B, int S_q, int S_kv, int D_qk, int D_v, float scale, float dropout,
                      bool causal, uint64 seed, uint64 offset) {
        return FromSdpa(sdpa_hip_fwd(dt, q, k, v, o, stats, B, S_q, S_kv, D_qk, D_v, scale, dropout, causal,
                                     seed, offset, stream(ctx)));
    }
    static Status bwd(OpKernelContext* ctx, int dt, const void* q, const void* k, const void* v, const void* o,
                      const float* stats, const void* d_o, void* dq, void* dk, void* dv, int B, int S_q,
                      int S_kv, int D_qk, int D_v, float scale, float dropout, bool causal, uint64 seed,
                      uint64 offset) {
        // Workspace from TF's allocator: the dS path's (the per-row values and
        // the stored dS, fp16 or fp32 at a feature size over 64) when it can be had,
        // else the per-row one (both backward kernels then form dS).
        size_t ws_bytes = sdpa_hip_bwd_workspace_bytes_ds(dt, B, S_q, S_kv, D_qk, D_v, causal ? 1 : 0);
        Tensor ws;
        Status st = ctx->allocate_temp(
            DT_UINT8, TensorShape({static_cast<int64_t>(std::max<size_t>(ws_bytes, 1))}), &ws);
        if (!st.ok()) {
            ws_bytes = sdpa_hip_bwd_workspace_bytes(B, S_q);
            TF_RETURN_IF_ERROR(ctx->allocate_temp(
                DT_UINT8, TensorShape({static_cast<int64_t>(std::max<size_t>(ws_bytes, 1))}), &ws));
        }
        return FromSdpa(sdpa_hip_bwd(dt, q, k, v, o, stats, d_o, dq, dk, dv, ws.flat<uint8>().data(), ws_bytes,
                                     B, S_q, S_kv, D_qk, D_v, scale, dropout, causal, seed, offset,
                                     stream(ctx)));
    }
};

}  // namespace

template <typename Device, typename T>
class SdpaFwdOp : public OpKernel {
 public:
    explicit SdpaFwdOp(OpKernelConstruction* c) : OpKernel(c) {
        OP_REQUIRES_OK(c, c->GetAttr("dropout", &dropout_));
        OP_REQUIRES_OK(c, c->GetAttr("scale", &scale_));
        OP_REQUIRES_OK(c, c->GetAttr("causal_mask", &causal_));
    }

    void Compute(OpKernelContext* ctx) override {
        const Tensor& q = ctx->input(0);
        const Tensor& k = ctx->input(1);
        const Tensor& v = ctx->input(2);
        const Tensor& seed = ctx->input(3);
        const Tensor& offset = ctx->input(4);
        const Dims qd(q), kd(k), vd(v);
        OP_REQUIRES_OK(ctx, FromSdpa(sdpa_hip_check_fwd(qd.rank, qd.d, kd.rank, kd.d, vd.rank, vd.d,
                                                        seed.dims(), offset.dims(), causal_)));
        const int B = qd.d[0], S_q = qd.d[1], D_qk = qd.d[2], S_kv = kd.d[1], D_v = vd.d[2];
        Tensor* o = nullptr;
        Tensor* stats = nullptr;
        OP_REQUIRES_OK(ctx, ctx->allocate_output(0, TensorShape({B, S_q, D_v}), &o));
        OP_REQUIRES_OK(ctx, ctx->allocate_output(1, TensorShape({B, S_q}), &stats));
        OP_REQUIRES_OK(ctx, Backend<Device>::fwd(ctx, dtype_code<T>(), q.flat<T>().data(), k.flat<T>().data(),
                                                 v.flat<T>().data(), o->flat<T>().data(),
                                                 stats->flat<float>().data(), B, S_q, S_kv, D_qk, D_v, scale_,
                                                 dropout_, causal_, seed.scalar<uint64>()(),
                                                 offset.scalar<uint64>()()));
    }

 private:
    float dropout_ = 0.f, scale_ = 1.f;
    bool causal_ = false;
};

template <typename Device, typename T>
class SdpaBwdOp : public OpKernel {
 public:
    explicit SdpaBwdOp(OpKernelConstruction* c) : OpKernel(c) {
        OP_REQUIRES_OK(c, c->GetAttr("dropout", &dropout_));
        OP_REQUIRES_OK(c, c->GetAttr("scale", &scale_));
        OP_REQUIRES_OK(c, c->GetAttr("causal_mask", &causal_));
    }

    void Compute(OpKernelContext* ctx) override {
        const Tensor& q = ctx->input(0);
        const Tensor& k = ctx->input(1);
        const Tensor& v = ctx->input(2);
        const Tensor& out = ctx->input(3);
        const Tensor& stats = ctx->input(4);
        const Tensor& d_o = ctx->input(5);
        const Tensor& seed = ctx->input(6);
        const Tensor& offset = ctx->input(7);
        const Dims qd(q), kd(k), vd(v), od(out), sd(stats), dd(d_o);
        OP_REQUIRES_OK(ctx, FromSdpa(sdpa_hip_check_bwd(qd.rank, qd.d, kd.rank, kd.d, vd.rank, vd.d, od.rank,
                                                        od.d, sd.rank, sd.d, dd.rank, dd.d, seed.dims(),
                                                        offset.dims(), causal_)));
        const int B = qd.d[0], S_q = qd.d[1], D_qk = qd.d[2], S_kv = kd.d[1], D_v = vd.d[2];
        Tensor* dq = nullptr;
        Tensor* dk = nullptr;
        Tensor* dv = nullptr;
        OP_REQUIRES_OK(ctx, ctx->allocate_output(0, q.shape(), &dq));
        OP_REQUIRES_OK(ctx, ctx->allocate_output(1, k.shape(), &dk));
        OP_REQUIRES_OK(ctx, ctx->allocate_output(2, v.shape(), &dv));
        OP_REQUIRES_OK(ctx, Backend<Device>::bwd(
                                ctx, dtype_code<T>(), q.flat<T>().data(), k.flat<T>().data(), v.flat<T>().data(),
                                out.flat<T>().data(), stats.flat<float>().data(), d_o.flat<T>().data(),
                                dq->flat<T>().data(), dk->flat<T>().data(), dv->flat<T>().data(), B, S_q, S_kv,
                                D_qk, D_v, scale_, dropout_, causal_, seed.scalar<uint64>()(),
                                offset.scalar<uint64>()()));
    }

 private:
    float dropout_ = 0.f, scale_ = 1.f;
    bool causal_ = false;
};

#define SDPA_REGISTER_CPU(T)                                                                     \
    REGISTER_KERNEL_BUILDER(Name("Sdpa").Device(DEVICE_CPU).TypeConstraint<T>("T"),              \
                            SdpaFwdOp<CPUDevice, T>);                                            \
    REGISTER_KERNEL_BUILDER(Name("SdpaGrad").Device(DEVICE_CPU).TypeConstraint<T>("T"),          \
                            SdpaBwdOp<CPUDevice, T>);
SDPA_REGISTER_CPU(float);
SDPA_REGISTER_CPU(Eigen::half);
#undef SDPA_REGISTER_CPU

#define SDPA_REGISTER_GPU(T)                                                                     \
    REGISTER_KERNEL_BUILDER(                                                                     \
        Name("Sdpa").Device(DEVICE_GPU).TypeConstraint<T>("T").HostMemory("seed").HostMemory("offset"), \
        SdpaFwdOp<GPUDevice, T>);                                                                \
    REGISTER_KERNEL_BUILDER(                                                                     \
        Name("SdpaGrad").Device(DEVICE_GPU).TypeConstraint<T>("T").HostMemory("seed").HostMemory("offset"), \
        SdpaBwdOp<GPUDevice, T>);
SDPA_REGISTER_GPU(float);
SDPA_REGISTER_GPU(Eigen::half);
#undef SDPA_REGISTER_GPU

}  // namespace tensorflow
