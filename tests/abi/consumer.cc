// A C++ caller of the two C ABIs (include/sdpa_hip.h, include/sdpa_cpu.h),
// built with g++ by tests/test_abi_consumers.py, the way a TensorFlow
// OpKernel includes them: the backward validation order and messages
// (sdpa/sdpa_cpu.cc:116-168), every status string, and the host backward
// kernel on a case with a closed form.  Exit status 0 on success.  No GPU
// work (the no-alloc entry point rejects an oversized problem on the host).
#include <array>
#include <cmath>
#include <cstdio>
#include <string>
#include <vector>

#include "sdpa_cpu.h"
#include "sdpa_hip.h"

#define CHECK(cond)                                                                   \
    do {                                                                              \
        if (!(cond)) {                                                                \
            std::fprintf(stderr, "check failed: %s (line %d)\n", #cond, __LINE__);    \
            return 1;                                                                 \
        }                                                                             \
    } while (0)

namespace {
int check_bwd(std::array<int64_t, 3> q, std::array<int64_t, 3> k, std::array<int64_t, 3> v,
              std::array<int64_t, 3> o, std::array<int64_t, 2> s, std::array<int64_t, 3> d_o) {
    return sdpa_hip_check_bwd(3, q.data(), 3, k.data(), 3, v.data(), 3, o.data(), 2, s.data(), 3,
                              d_o.data(), 0, 0, 0);
}
}  // namespace

int main() {
    const std::array<int64_t, 3> q{2, 4, 8}, k{2, 6, 8}, v{2, 6, 5}, o{2, 4, 5}, d_o{2, 4, 5};
    const std::array<int64_t, 2> s{2, 4};
    CHECK(check_bwd(q, k, v, o, s, d_o) == SDPA_OK);
    CHECK(std::string(sdpa_hip_status_string(check_bwd(q, k, v, {2, 5, 5}, s, d_o))) == "O seq size mismatch");
    CHECK(std::string(sdpa_hip_status_string(check_bwd(q, k, v, o, s, {2, 4, 4}))) == "dO feature size mismatch");
    CHECK(std::string(sdpa_hip_status_string(check_bwd(q, k, v, o, {2, 7}, d_o))) == "S seq size mismatch");
    // the first failing check wins, in the reference's order (K before O)
    CHECK(check_bwd(q, {2, 6, 7}, v, {9, 9, 9}, s, d_o) == SDPA_ERR_K_FEATURE);
    for (int code = 0; code <= SDPA_ERR_SCRATCH_LIMIT; ++code) CHECK(sdpa_hip_status_string(code)[0] != '\0');
    CHECK(sdpa_hip_bwd_noalloc(SDPA_DTYPE_F16, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr,
                               nullptr, nullptr, 1, 1 << 22, 1 << 22, 8, 8, 1.f, 0.f, 0, 0, 0,
                               nullptr) == SDPA_ERR_SCRATCH_LIMIT);

    // host backward with one key: P = 1 exactly (stats = s, scale 1), so
    // dV = sum_i dO_i, dP_i = dO_i . v, delta_i = dO_i . o_i, dS_i = dP_i - delta_i,
    // dK = sum_i dS_i q_i, dQ_i = dS_i k
    const int B = 1, S_q = 3, S_kv = 1, D = 2;
    std::vector<float> qv{1, 2, 3, 4, 5, 6}, kv{0.5f, -1}, vv{2, 3}, ov(S_q * D, 0.f), dov{1, 0, 0, 1, 1, 1};
    std::vector<float> st(S_q), dq(S_q * D), dk(D), dv(D);
    for (int i = 0; i < S_q; ++i) st[i] = qv[2 * i] * kv[0] + qv[2 * i + 1] * kv[1];
    int rc = sdpa_cpu_bwd(SDPA_CPU_DTYPE_F32, qv.data(), kv.data(), vv.data(), ov.data(), st.data(), dov.data(),
                          dq.data(), dk.data(), dv.data(), B, S_q, S_kv, D, D, 1.f, 0.f, 0, 0, 0, 2);
    CHECK(rc == SDPA_OK);
    CHECK(std::fabs(dv[0] - 2.f) < 1e-6f && std::fabs(dv[1] - 2.f) < 1e-6f);
    const float ds[3] = {2.f, 3.f, 5.f};  // dO_i . v with o = 0
    CHECK(std::fabs(dk[0] - (ds[0] * 1 + ds[1] * 3 + ds[2] * 5)) < 1e-5f);
    CHECK(std::fabs(dk[1] - (ds[0] * 2 + ds[1] * 4 + ds[2] * 6)) < 1e-5f);
    for (int i = 0; i < S_q; ++i) CHECK(std::fabs(dq[2 * i] - ds[i] * 0.5f) < 1e-6f && std::fabs(dq[2 * i + 1] + ds[i]) < 1e-6f);
    std::printf("consumer.cc ok\n");
    return 0;
}
