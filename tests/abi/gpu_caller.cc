// A C++ host program that drives the GPU forward and backward through the C
// ABI (include/sdpa_hip.h) with its own HIP allocations and stream, as an
// OpKernel does: device buffers from hipMalloc, the backward workspace sized
// by sdpa_hip_bwd_workspace_bytes, launches on a stream it created.
//
//   gpu_caller DIR dtype B S_q S_kv D_qk D_v causal dropout scale seed offset
//
// reads DIR/{q,k,v,do}.bin (raw little-endian tensors of the dtype) and
// writes DIR/{o,stats,dq,dk,dv}.bin; tests/test_abi_consumers.py compares
// them with the CPU oracle.  Built by __graft_entry__.build() with g++
// against the HIP runtime.
#include <hip/hip_runtime_api.h>

#include <cstdio>
#include <cstdlib>
#include <fstream>
#include <string>
#include <vector>

#include "sdpa_hip.h"

namespace {
bool hip_ok(hipError_t e, const char* what) {
    if (e == hipSuccess) return true;
    std::fprintf(stderr, "%s: %s\n", what, hipGetErrorString(e));
    return false;
}

std::vector<char> read_file(const std::string& path, size_t bytes) {
    std::vector<char> buf(bytes);
    std::ifstream f(path, std::ios::binary);
    if (!f.read(buf.data(), (std::streamsize)bytes)) buf.clear();
    return buf;
}

bool write_file(const std::string& path, const std::vector<char>& buf) {
    std::ofstream f(path, std::ios::binary);
    return (bool)f.write(buf.data(), (std::streamsize)buf.size());
}
}  // namespace

int main(int argc, char** argv) {
    if (argc != 13) {
        std::fprintf(stderr, "usage: %s DIR dtype B S_q S_kv D_qk D_v causal dropout scale seed offset\n", argv[0]);
        return 2;
    }
    const std::string dir = argv[1];
    const int dtype = std::atoi(argv[2]), B = std::atoi(argv[3]), S_q = std::atoi(argv[4]),
              S_kv = std::atoi(argv[5]), D_qk = std::atoi(argv[6]), D_v = std::atoi(argv[7]),
              causal = std::atoi(argv[8]);
    const float dropout = std::strtof(argv[9], nullptr), scale = std::strtof(argv[10], nullptr);
    const uint64_t seed = std::strtoull(argv[11], nullptr, 10), offset = std::strtoull(argv[12], nullptr, 10);
    const size_t es = dtype == SDPA_DTYPE_F16 ? 2 : 4;
    const size_t nq = (size_t)B * S_q * D_qk * es, nk = (size_t)B * S_kv * D_qk * es,
                 nv = (size_t)B * S_kv * D_v * es, no = (size_t)B * S_q * D_v * es,
                 ns = (size_t)B * S_q * sizeof(float);

    struct Buf {
        const char* name;
        size_t bytes;
        void* dev;
    } bufs[] = {{"q", nq, nullptr},  {"k", nk, nullptr},     {"v", nv, nullptr},   {"do", no, nullptr},
                {"o", no, nullptr},  {"stats", ns, nullptr}, {"dq", nq, nullptr},  {"dk", nk, nullptr},
                {"dv", nv, nullptr}};
    for (auto& b : bufs)
        if (!hip_ok(hipMalloc(&b.dev, b.bytes ? b.bytes : 1), "hipMalloc")) return 1;
    for (int i = 0; i < 4; ++i) {
        std::vector<char> h = read_file(dir + "/" + bufs[i].name + ".bin", bufs[i].bytes);
        if (h.size() != bufs[i].bytes) {
            std::fprintf(stderr, "cannot read %s.bin\n", bufs[i].name);
            return 1;
        }
        if (!hip_ok(hipMemcpy(bufs[i].dev, h.data(), h.size(), hipMemcpyHostToDevice), "hipMemcpy")) return 1;
    }
    hipStream_t stream = nullptr;
    if (!hip_ok(hipStreamCreate(&stream), "hipStreamCreate")) return 1;
    const size_t ws_bytes = sdpa_hip_bwd_workspace_bytes(B, S_q);
    void* ws = nullptr;
    if (!hip_ok(hipMalloc(&ws, ws_bytes ? ws_bytes : 1), "hipMalloc")) return 1;

    int rc = sdpa_hip_fwd(dtype, bufs[0].dev, bufs[1].dev, bufs[2].dev, bufs[4].dev, (float*)bufs[5].dev, B, S_q,
                          S_kv, D_qk, D_v, scale, dropout, causal, seed, offset, stream);
    if (rc != SDPA_OK) {
        std::fprintf(stderr, "sdpa_hip_fwd: %s\n", sdpa_hip_status_string(rc));
        return 1;
    }
    rc = sdpa_hip_bwd(dtype, bufs[0].dev, bufs[1].dev, bufs[2].dev, bufs[4].dev, (const float*)bufs[5].dev,
                      bufs[3].dev, bufs[6].dev, bufs[7].dev, bufs[8].dev, ws, ws_bytes, B, S_q, S_kv, D_qk, D_v,
                      scale, dropout, causal, seed, offset, stream);
    if (rc != SDPA_OK) {
        std::fprintf(stderr, "sdpa_hip_bwd: %s\n", sdpa_hip_status_string(rc));
        return 1;
    }
    if (!hip_ok(hipStreamSynchronize(stream), "hipStreamSynchronize")) return 1;
    for (int i = 4; i < 9; ++i) {
        std::vector<char> h(bufs[i].bytes);
        if (!hip_ok(hipMemcpy(h.data(), bufs[i].dev, h.size(), hipMemcpyDeviceToHost), "hipMemcpy")) return 1;
        if (!write_file(dir + "/" + bufs[i].name + ".bin", h)) return 1;
    }
    bool ok = hip_ok(hipStreamDestroy(stream), "hipStreamDestroy") && hip_ok(hipFree(ws), "hipFree");
    for (auto& b : bufs) ok = hip_ok(hipFree(b.dev), "hipFree") && ok;
    if (!ok) return 1;
    std::printf("gpu_caller ok\n");
    return 0;
}
