// sdpa_f32_dq_ds.hip -- the dS path of the fp32 SdpaGrad for gfx950: dQ as a
// product with the dS the fp32 split dK/dV kernel stored (DsLayout32), instead
// of the dQ kernel that forms S, P, dP and dS once more (sdpa_bwd.hip).
//
// Order of the path (sdpa_capi.hip):
//   1. row kernel  -- delta (and stats2) per query row into the workspace, as
//                     the other path's dQ kernel writes them first;
//   2. dK/dV       -- sdpa_bwd_dkdv_f32_split_kernel with p.ds set: its dS
//                     role stores every dS it forms;
//   3. dQ          -- dQ^T = K^T dS^T per 32 queries, scaled once at the store.
// In fp32 the products run on v_mfma_f32_32x32x2_f32, so dQ stays bound by
// its one product (the recomputing kernel executes three).
//
// Element semantics (sdpa/sdpa_bwd.cu.cc:291-327): dQ_i = scale sum_j dS_ij
// K_j with dS as the dK/dV kernel forms it (P gated at 1e-6, the dropout
// decision, dP scaled by 1/(1-p) for kept elements).
#include <type_traits>

#include "sdpa_dma.h"
#include "sdpa_launch.h"
#include "sdpa_params.h"

namespace sdpa {
namespace {

// ---------------------------------------------------------------------------
// Row values.  Lane = query row, hh = half of the features: delta = sum_d dO
// O summed as the fp32 dQ kernel's prologue sums it (its lane, feature and
// fma order), so that both paths hand the dK/dV kernel the same delta and dK,
// dV are bit-identical between them.  stats2 as that prologue writes it.
// ---------------------------------------------------------------------------
template <int DV>
__global__ __launch_bounds__(256) void sdpa_bwd_rows_f32_kernel(const BwdParams p) {
    constexpr int HV = DV / 2;
    const int tid = threadIdx.x, lane = tid & 63, l32 = lane & 31, hh = lane >> 5, wave = tid >> 6;
    const int S_q = p.s.S_q, D_v = p.s.D_v;
    const int tiles = (S_q + 127) / 128;
    const int b = (int)(blockIdx.x / (unsigned)tiles), qt = (int)(blockIdx.x % (unsigned)tiles);
    const int my_q = qt * 128 + 32 * wave + l32;
    const size_t row_q = (size_t)b * S_q + my_q;
    const float* Ob = static_cast<const float*>(p.o) + (size_t)b * S_q * D_v;
    const float* dOb = static_cast<const float*>(p.d_o) + (size_t)b * S_q * D_v;
    float dpart = 0.f;
#pragma unroll
    for (int u = 0; u < HV / 4; ++u) {
        const floatx4 f = __builtin_bit_cast(floatx4, load_row_chunk<float, true>(dOb, my_q, S_q, HV * hh + 4 * u, D_v, D_v));
        const floatx4 o = __builtin_bit_cast(floatx4, load_row_chunk<float, true>(Ob, my_q, S_q, HV * hh + 4 * u, D_v, D_v));
#pragma unroll
        for (int e = 0; e < 4; ++e) dpart += f[e] * o[e];
    }
    const float delta = xhalf_sum(dpart);
    if (my_q < S_q && hh == 0) {
        const float stats2 = p.stats[row_q] * kLog2e;
        p.delta[row_q] = delta;
        p.stats2[row_q] = stats2 + kGateShift;
    }
}

// ---------------------------------------------------------------------------
// dQ from the stored dS.  Four waves of 32 queries (128 per workgroup): a
// wave owns one stored query block.  Key steps of 32 (one stored key group)
// through two LDS stages of the K tile (32 rows of D_qk floats, row-major)
// and each wave's dS tile (one stored 4 KB key group, copied as it lies).  Each
// v_mfma_f32_32x32x2_f32 takes a key pair: lane (l32, hh) reads
// K[2 p + hh][32 dt + l32] (the A operand K^T) and dS[2 p + hh][l32] (the B
// operand dS^T, lane = query position), so the accumulators hold dQ^T with
// lane = query position, and lane l32 stores query pi(l32) of the block.
// ---------------------------------------------------------------------------
template <int DQK>
struct DqDs32Cfg {
    static constexpr int NW = 4, NT = 64 * NW, BM = 32 * NW, BN = 32, NSTAGE = 2;
    static constexpr int LK = DQK / 4;           // 16-byte chunks per K row
    static constexpr int KB = BN * DQK * 4;      // K tile
    static constexpr int SB = BN * 32 * 4;       // one wave's dS tile (4 KB)
    static constexpr int CPW = KB / 1024 / NW;   // K copies of 1 KB per wave
    static constexpr int STAGE = KB + NW * SB;
    static constexpr size_t LDS_BYTES = NSTAGE * (size_t)STAGE;
    static_assert(CPW >= 1 && KB % (1024 * NW) == 0, "every wave copies whole KB of the K tile");
    static_assert(2 * LDS_BYTES <= 160 * 1024, "two workgroups per CU");
};

template <int DQK, bool CAUSAL>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2)))
void sdpa_bwd_dq_ds_f32_kernel(const BwdParams p, const int win) {
    using Cfg = DqDs32Cfg<DQK>;
    constexpr int BM = Cfg::BM, BN = Cfg::BN, LK = Cfg::LK, NSTAGE = Cfg::NSTAGE, CPW = Cfg::CPW;
    constexpr int NDT = DQK / 32;
    static_assert(DsLayout32::KT % BN == 0 && BN == DsLayout32::QBK, "steps tile the stored key groups");
    static_assert(NSTAGE == 2, "one step of copies ahead");

    const int tid = threadIdx.x, lane = tid & 63, l32 = lane & 31, hh = lane >> 5;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int B = p.s.B, S_q = p.s.S_q, S_kv = p.s.S_kv, D_qk = p.s.D_qk;
    const int tiles = (S_q + BM - 1) / BM;
    int b, qt;
    xcd_map(blockIdx.x, B * tiles, tiles, CAUSAL, win, b, qt);
    const int qw0 = qt * BM + 32 * wave, qb = qw0 / DsLayout32::QBK;
    const int pq = 8 * ((l32 >> 2) & 3) + 4 * (l32 >> 4) + (l32 & 3);  // stored position -> query
    const DsLayout32 dsl(S_q, S_kv, CAUSAL);
    const unsigned char* dsb = static_cast<const unsigned char*>(p.ds);

    // The dK/dV kernel stored this wave's block at the key group kv0 under
    // the same predicate (its `live`).
    auto live = [&](int kv0) { return qw0 < S_q && kv0 < S_kv && !(CAUSAL && qw0 + 31 < kv0); };

    // K tile copies: copy u of wave w fills LDS bytes (CPW w + u) KB + 16
    // lane, i.e. chunk slot s = 64 (CPW w + u) + lane: row s / LK, slot
    // s % LK.  Odd rows hold chunk slot ^ 8 (D_qk >= 64), so the two rows of
    // a key pair, 256 or 512 bytes apart, fall in different bank halves.
    constexpr int SWZ = DQK >= 64 ? 8 : 0;
    const RowSrc ksrc = row_src(p.k, (size_t)b * S_kv, S_kv, D_qk * 4);
    uint32_t kvoff[CPW];
#pragma unroll
    for (int u = 0; u < CPW; ++u) {
        const int s = 64 * (CPW * wave + u) + lane, r = s / LK;
        const int c = (s % LK) ^ ((r & 1) ? SWZ : 0);
        kvoff[u] = c < D_qk / 4 ? (uint32_t)(r * D_qk * 4 + c * 16) : kOob;
    }
    const uint32_t lds0 = lds_base();
    const int kv_end = CAUSAL ? min(S_kv, qt * BM + BM) : S_kv;
    const int nsteps = (kv_end + BN - 1) / BN;
    // copies of step `step` into stage step % 2: the wave's share of the K
    // tile and, when its block is live there, its dS tile (4 KB)
    auto issue = [&](int step) {
        const int kv0 = step * BN;
        const uint32_t so = (uint32_t)((step % NSTAGE) * Cfg::STAGE);
        const rsrc_t rk = ksrc.shifted(kv0).at(0);
#pragma unroll
        for (int u = 0; u < CPW; ++u) dma16_at(rk, lds0 + so + 1024u * (uint32_t)(CPW * wave + u), kvoff[u]);
        if (live(kv0)) {
            const unsigned char* src =
                dsb + dsl.offset(b, kv0 / DsLayout32::KT, qb) + ((kv0 % DsLayout32::KT) / 32) * 4096;
            // dS is read once: non-temporal
            const rsrc_t rs = RowSrc{uniform_ptr(src), 32, 128, 0x7FFFFFFF / 128}.at(0);
            const uint32_t m0 = lds0 + so + (uint32_t)(Cfg::KB + Cfg::SB * wave);
#pragma unroll
            for (int u = 0; u < 4; ++u) dma16_at_nt(rs, m0 + 1024u * u, (uint32_t)(16 * lane + 1024 * u));
        }
    };

    floatx16 acc[NDT];
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) acc[dt] = floatx16{};
    // lane terms of the reads: K[2 p + hh][32 dt + l32] and dS[2 p + hh][l32].
    // dS sits at DsLayout32::slot32(2 p + hh, l32), with u = (l32 >> 2) & 3
    // and h = l32 >> 4 from the lane's query position; for p = 4 i + j its
    // key slot is 8 i + ((2 j + hh) ^ (u + 4 h)) (the XOR term stays below 8),
    // so one lane base per j and the immediate 128 i.
    const int krow_sw = hh ? SWZ : 0;
    int sbase[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) sbase[j] = DsLayout32::slot32(2 * j + hh, l32);
    // All of a step's operands are read first (BN / 2 (1 + NDT) floats per
    // lane), so that each MFMA finds its operands landed instead of waiting
    // out the LDS latency of a read issued just before it.
    auto step_mfma = [&](uint32_t so) {
        const float* Ks = reinterpret_cast<const float*>(smem + so);
        const unsigned char* Ss = smem + so + Cfg::KB + Cfg::SB * wave;
        float bv[BN / 2], av[BN / 2][NDT];
#pragma unroll
        for (int pr = 0; pr < BN / 2; ++pr) {
            const int r = 2 * pr + hh;
            bv[pr] = *reinterpret_cast<const float*>(Ss + sbase[pr & 3] + 128 * (pr >> 2));
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt) {
                const int c = (8 * dt + (l32 >> 2)) ^ krow_sw;
                av[pr][dt] = Ks[r * DQK + 4 * c + (l32 & 3)];
            }
        }
#pragma unroll
        for (int pr = 0; pr < BN / 2; ++pr)
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt) acc[dt] = mfma_f32(av[pr][dt], bv[pr], acc[dt]);
    };

    if (nsteps > 0) issue(0);
    for (int step = 0; step < nsteps; ++step) {
        wait_vm();
        __syncthreads();
        // stage (step + 1) % 2 held step - 1, which every wave has finished
        if (step + 1 < nsteps) issue(step + 1);
        if (live(step * BN)) step_mfma((uint32_t)((step % NSTAGE) * Cfg::STAGE));
    }

    const int my_q = qw0 + pq;
    if (my_q < S_q) {
        const float f = p.c.scale;
        float* dQb = static_cast<float*>(p.dq) + ((size_t)b * S_q + my_q) * D_qk;
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
            for (int g4 = 0; g4 < 4; ++g4) {
                const int d0 = 32 * dt + 8 * g4 + 4 * hh;
                floatx4 fv;
#pragma unroll
                for (int e = 0; e < 4; ++e) fv[e] = acc[dt][4 * g4 + e] * f;
                if (d0 < D_qk) *reinterpret_cast<floatx4*>(dQb + d0) = fv;
            }
    }
}

}  // namespace

hipError_t launch_bwd_rows_f32(const BwdParams& p, hipStream_t stream) {
    const int B = p.s.B, S_q = p.s.S_q;
    if (B == 0 || S_q == 0) return hipSuccess;
    const long long n = (long long)((S_q + 127) / 128) * B;
    if (n > 0x7FFFFFFFLL) return hipErrorInvalidValue;
    return with_dim(p.s.D_v, [&](auto dv) {
        constexpr int DV = decltype(dv)::value;
        return launch_kernel<sdpa_bwd_rows_f32_kernel<DV>>((unsigned)n, 256, 0, stream, p);
    });
}

hipError_t launch_bwd_dq_ds_f32(const BwdParams& p, hipStream_t stream) {
    const int B = p.s.B, S_q = p.s.S_q;
    if (B == 0 || S_q == 0) return hipSuccess;
    if (!p.ds) return hipErrorInvalidValue;
    return with_dim(p.s.D_qk, [&](auto dqk) {
        return with_bool(p.c.causal != 0, [&](auto c) {
            constexpr int DQK = decltype(dqk)::value;
            using Cfg = DqDs32Cfg<DQK>;
            const long long n = (long long)((S_q + Cfg::BM - 1) / Cfg::BM) * B;
            return launch_kernel<sdpa_bwd_dq_ds_f32_kernel<DQK, decltype(c)::value>>(
                (unsigned)n, Cfg::NT, Cfg::LDS_BYTES, stream, p, row_window((size_t)p.s.S_kv * DQK * 4));
        });
    });
}

}  // namespace sdpa
