/* A plain C caller of the two C ABIs (include/sdpa_hip.h, include/sdpa_cpu.h),
 * built with gcc by tests/test_abi_consumers.py: the headers compile as C
 * without any HIP header, the validation entry points return the
 * reference's codes and messages (sdpa/sdpa_cpu.cc:37-69), and the host
 * forward kernel runs.  Exit status 0 on success; the failing check is
 * printed otherwise.  No GPU work. */
#include <math.h>
#include <stdio.h>
#include <string.h>

#include "sdpa_cpu.h"
#include "sdpa_hip.h"

#define CHECK(cond)                                              \
    do {                                                         \
        if (!(cond)) {                                           \
            fprintf(stderr, "check failed: %s (line %d)\n", #cond, __LINE__); \
            return 1;                                            \
        }                                                        \
    } while (0)

int main(void) {
    const int64_t q[3] = {2, 4, 8}, k[3] = {2, 6, 8}, v[3] = {2, 6, 5}, kbad[3] = {3, 6, 8};
    int rc = sdpa_hip_check_fwd(3, q, 3, k, 3, v, 0, 0, 0);
    CHECK(rc == SDPA_OK);
    rc = sdpa_hip_check_fwd(3, q, 3, k, 3, v, 0, 0, 1);
    CHECK(rc == SDPA_ERR_CAUSAL_SEQ);
    CHECK(strcmp(sdpa_hip_status_string(rc), "seq size Q != K while causal_mask = True") == 0);
    rc = sdpa_hip_check_fwd(3, q, 3, kbad, 3, v, 0, 0, 0);
    CHECK(strcmp(sdpa_hip_status_string(rc), "K batch size mismatch") == 0);
    rc = sdpa_hip_check_fwd(3, q, 3, k, 3, v, 1, 0, 0);
    CHECK(strcmp(sdpa_hip_status_string(rc), "seed must be scalar") == 0);
    rc = sdpa_hip_check_fwd(2, q, 3, k, 3, v, 0, 0, 0);
    CHECK(strcmp(sdpa_hip_status_string(rc), "Shape must be rank 3") == 0);
    CHECK(sdpa_hip_drop_threshold(0.1f) == 0x19999991u);
    CHECK(sdpa_hip_bwd_workspace_bytes(128, 4096) == (size_t)2 * 128 * 4096 * 4);

    /* host forward, q = 0: every key has the same score, o = mean of v */
    enum { B = 1, S = 3, D = 4 };
    float qz[B * S * D] = {0}, kk[B * S * D], vv[B * S * D], o[B * S * D], st[B * S];
    for (int i = 0; i < B * S * D; ++i) {
        kk[i] = (float)(i % 5) - 2.0f;
        vv[i] = (float)i;
    }
    rc = sdpa_cpu_fwd(SDPA_CPU_DTYPE_F32, qz, kk, vv, o, st, B, S, S, D, D, 0.5f, 0.0f, 0, 0, 0, 1);
    CHECK(rc == SDPA_OK);
    for (int i = 0; i < S; ++i)
        for (int d = 0; d < D; ++d) CHECK(fabsf(o[i * D + d] - (vv[d] + vv[D + d] + vv[2 * D + d]) / 3.0f) < 1e-5f);
    CHECK(fabsf(st[0] - logf(3.0f + 1e-6f)) < 1e-6f);
    printf("consumer.c ok\n");
    return 0;
}
