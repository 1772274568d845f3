// sdpa_f16_dq.hip -- fp16 SdpaGrad dQ kernel for gfx950 that streams its K/V
// tiles from HBM straight into LDS (copy machinery in sdpa_dma.h).  It runs
// first in the backward and leaves stats2 and delta in the workspace for the
// dK/dV kernel (sdpa_f16_dkdv.hip).
//
// The production dQ kernel for the fp16 op whenever every feature width is a
// multiple of 8 and every tensor is 16-byte aligned; other fp16 shapes use
// the register-staged kernel of sdpa_bwd.hip.  Element semantics are those of
// the reference (sdpa/sdpa_bwd.cu.cc:291-327), restated in sdpa_bwd.hip.
//
// Per wave of 32 queries (lane = query), v_mfma_f32_32x32x16_f16 with fp32
// accumulation (lane layouts in sdpa_device.h):
//   S^T = K Q^T, dP^T = V dO^T, dQ^T += K^T dS^T.
// Two LDS stages: the copy of step n + 1 is in flight while step n is
// multiplied, one barrier per step.  Workgroup ids are remapped XCD-major
// (xcd_map).
#include <type_traits>

#include "sdpa_dma.h"
#include "sdpa_launch.h"
#include "sdpa_params.h"

namespace sdpa {
namespace {

// ===========================================================================
// Backward, dQ kernel (also writes stats2 and delta to the workspace)
// ===========================================================================
template <int DQK, int DV>
struct DqDmaCfg {
    static constexpr int NT = 256, BM = 128, BN = 64;
    static constexpr int LK = DQK / 8, LV = DV / 8;
    static constexpr int KB = BN * DQK * 2, VB = BN * DV * 2, STAGE = KB + VB;
    static constexpr size_t LDS_BYTES = 2 * (size_t)STAGE;
    // waves per SIMD: three for D <= 64 without dropout (registers under 168)
    template <bool DROP>
    static constexpr int wpe() { return (!DROP && DQK <= 64 && DV <= 64 && 3 * LDS_BYTES <= 160 * 1024) ? 3 : 2; }
};

template <int DQK, int DV, bool CAUSAL, bool DROP>
__global__ __launch_bounds__(256)
__attribute__((amdgpu_waves_per_eu(DqDmaCfg<DQK, DV>::template wpe<DROP>(), DqDmaCfg<DQK, DV>::template wpe<DROP>())))
void sdpa_bwd_dq_f16_dma_kernel(const BwdParams p, const int win) {
    using Cfg = DqDmaCfg<DQK, DV>;
    constexpr int BM = Cfg::BM, BN = Cfg::BN, LK = Cfg::LK, LV = Cfg::LV;

    const int tid = threadIdx.x, lane = tid & 63, l32 = lane & 31, hh = lane >> 5;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int B = p.s.B, S_q = p.s.S_q, S_kv = p.s.S_kv, D_qk = p.s.D_qk, D_v = p.s.D_v;
    const int tiles = (S_q + BM - 1) / BM;
    int b, qt;
    xcd_map(blockIdx.x, B * tiles, tiles, CAUSAL, win, b, qt);
    const int q0 = qt * BM, qw0 = q0 + 32 * wave, my_q = qw0 + l32;
    const size_t row_q = (size_t)b * S_q + my_q;

    const half_t* Qb = static_cast<const half_t*>(p.q) + (size_t)b * S_q * D_qk;
    const half_t* Ob = static_cast<const half_t*>(p.o) + (size_t)b * S_q * D_v;
    const half_t* dOb = static_cast<const half_t*>(p.d_o) + (size_t)b * S_q * D_v;
    const half_t* Kb = static_cast<const half_t*>(p.k) + (size_t)b * S_kv * D_qk;
    const half_t* Vb = static_cast<const half_t*>(p.v) + (size_t)b * S_kv * D_v;

    half8 qreg[DQK / 16], doreg[DV / 16];
#pragma unroll
    for (int ks = 0; ks < DQK / 16; ++ks)
        qreg[ks] = __builtin_bit_cast(half8, load_row_chunk<half_t, true>(Qb, my_q, S_q, 16 * ks + 8 * hh, D_qk, D_qk));
    float dpart = 0.f;
#pragma unroll
    for (int ks = 0; ks < DV / 16; ++ks) {
        doreg[ks] = __builtin_bit_cast(half8, load_row_chunk<half_t, true>(dOb, my_q, S_q, 16 * ks + 8 * hh, D_v, D_v));
        const half8 o8 = __builtin_bit_cast(half8, load_row_chunk<half_t, true>(Ob, my_q, S_q, 16 * ks + 8 * hh, D_v, D_v));
#pragma unroll
        for (int e = 0; e < 8; ++e) dpart += (float)doreg[ks][e] * (float)o8[e];
    }
    const float delta = xhalf_sum(dpart);
    const bool row_ok = my_q < S_q;
    // stats * log2(e) + kGateShift with one rounding (an explicit fma: left
    // to contraction, the rounding depended on the code around it)
    const float stats2g = row_ok ? __builtin_fmaf(p.stats[row_q], kLog2e, kGateShift) : INFINITY;
    if (row_ok && hh == 0) {
        p.delta[row_q] = delta;
        p.stats2[row_q] = stats2g;
    }
    const float sl2 = p.c.scale_log2;
    // P' = exp2(S sl2 - stats2 - kGateShift) is 0 where P <= 1e-6 and P / 2^kGateShift
    // elsewhere: dS = P' (keep ? dP (1/(1-p)) - delta : -delta) 2^kGateShift, the
    // factor taken into the two per-row constants.
    const float nst = -stats2g;
    const float kscg = p.c.keep_scale * kGateScale;
    const float deltag = delta * kGateScale;

    TileDma<BN, LK, 4> kd;
    TileDma<BN, LV, 4> vd;
    kd.init(wave, lane, D_qk * 2, D_qk / 8);
    vd.init(wave, lane, D_v * 2, D_v / 8);
    const int kv_end = CAUSAL ? min(S_kv, q0 + BM) : S_kv;
    const int nsteps = (kv_end + BN - 1) / BN;
    auto issue = [&](int step) {
        const int kv0 = step * BN;
        unsigned char* st = smem + (step & 1) * Cfg::STAGE;
        kd.issue(make_rsrc(Kb + (size_t)kv0 * D_qk, (long long)(S_kv - kv0) * D_qk * 2), st, wave);
        vd.issue(make_rsrc(Vb + (size_t)kv0 * D_v, (long long)(S_kv - kv0) * D_v * 2), st + Cfg::KB, wave);
    };
    if (nsteps > 0) issue(0);

    const uint64_t st_lane = DROP ? lcg_state(p.c.seed_offset, row_q, (uint64_t)S_kv, 4 * hh) : 0;
    const uint32_t thr = p.c.drop_threshold;

    SwzLane<LK> swK;
    SwzLane<LV> swV;
    swK.init(lane);
    swV.init(lane);

    floatx16 dqacc[DQK / 32];
#pragma unroll
    for (int dt = 0; dt < DQK / 32; ++dt) dqacc[dt] = floatx16{};

    // dS of one 32-key sub-tile; the rows of the accumulators are keys
    // k0 + 8 (r/4) + 4 hh + r%4.  PART: the causal mask or the key tail cuts it.
    auto elem = [&]<bool PART>(const floatx16& sacc, const floatx16& dpacc, int k0, half8& ds0, half8& ds1) {
        uint64_t st_blk = DROP ? st_lane + (uint64_t)k0 * kLcgMul : 0;
        // hash states after the MFMAs (hoisted above them they hold 32 VGPRs)
        if constexpr (DROP) asm volatile("" : "+v"(st_blk) : "v"(dpacc[15]));
        uint32_t w[8];
#pragma unroll
        for (int r = 0; r < 16; r += 2) {
            float ds2[2];
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const int rr = r + e;
                float x = __builtin_fmaf(sacc[rr], sl2, nst);
                if constexpr (PART) {
                    const int key = k0 + 8 * (rr >> 2) + 4 * hh + (rr & 3);
                    if (key >= S_kv || (CAUSAL && key > my_q)) x = -INFINITY;
                }
                const float pg = fast_exp2(x);  // P', gated
                float tt;
                if constexpr (DROP) {
                    const bool keep = lcg_keep(st_blk + (uint64_t)(8 * (rr >> 2) + (rr & 3)) * kLcgMul, thr);
                    tt = keep ? __builtin_fmaf(dpacc[rr], kscg, -deltag) : -deltag;
                } else {
                    tt = __builtin_fmaf(dpacc[rr], kscg, -deltag);  // kscg = 2^kGateShift here
                }
                ds2[e] = pg * tt;
            }
            w[r >> 1] = pack_h2(ds2[0], ds2[1]);
            // without dropout the compiler otherwise runs the exponentials
            // far ahead and spills at D = 128 (the copy offsets, whose
            // reloads then wait for the copies in flight)
            if constexpr (!DROP) __builtin_amdgcn_sched_barrier(0);
        }
        ds0 = half8_of(w[0], w[1], w[2], w[3]);
        ds1 = half8_of(w[4], w[5], w[6], w[7]);
    };
    // Sub-tile t of the step at kbase.  The S and dP chains read their A
    // operands RD MFMAs ahead, and scheduling fences keep the reads there
    // (left to itself the compiler reads each operand just before its MFMA
    // and waits out the whole LDS latency every time); the transposed reads
    // for dQ go out before the element-wise work and land during it.
    constexpr int NK = DQK / 16, NV = DV / 16, RD_FULL = SDPA_RD;
    auto sub = [&]<bool PART>(uint32_t kbase, int k0, int t, auto&& after_chains) {
        // masked sub-tiles read one operand ahead: their mask code needs the
        // registers (RD ahead spills at D = 128)
        constexpr int RD = PART ? 1 : RD_FULL;
        const uint32_t aK = kbase + swK.row, aV = kbase + Cfg::KB + swV.row;
        const uint32_t aK0 = kbase + swK.tr0, aK1 = kbase + swK.tr1;
        auto rd = [&](int i) { return i < NK ? lds_row<LK>(aK, i, 32 * t) : lds_row<LV>(aV, i - NK, 32 * t); };
        half8 op[NK + NV];
#pragma unroll
        for (int i = 0; i < RD; ++i) op[i] = rd(i);
        __builtin_amdgcn_sched_barrier(0);
        floatx16 sacc = floatx16{}, dpacc = floatx16{};
#pragma unroll
        for (int i = 0; i < NK + NV; ++i) {
            if (i + RD < NK + NV) op[i + RD] = rd(i + RD);
            if (i < NK) sacc = mfma_f16(op[i], qreg[i], sacc);
            else dpacc = mfma_f16(op[i], doreg[i - NK], dpacc);
            __builtin_amdgcn_sched_barrier(0);
        }
        after_chains();
        __builtin_amdgcn_sched_barrier(0);
        half8 at[2][DQK / 32];
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int dt = 0; dt < DQK / 32; ++dt) at[j][dt] = lds_tr<LK>(aK0, aK1, dt, 32 * t + 16 * j);
        __builtin_amdgcn_sched_barrier(0);
        half8 ds0, ds1;
        elem.template operator()<PART>(sacc, dpacc, k0, ds0, ds1);
#pragma unroll
        for (int dt = 0; dt < DQK / 32; ++dt) {
            dqacc[dt] = mfma_f16(at[0][dt], ds0, dqacc[dt]);
            dqacc[dt] = mfma_f16(at[1][dt], ds1, dqacc[dt]);
        }
    };
    auto sync_step = [&](int step) {
        wait_vm();
        __syncthreads();
        if (step + 1 < nsteps) issue(step + 1);
    };
    auto none = [] {};
    // Steps whose 64 keys are all visible to all 32 queries of the wave come
    // first (no mask code); the causal diagonal and the key tail follow, every
    // live sub-tile through the masked path (with the unmasked path as well,
    // the loop merged the dQ accumulators of the two with 130 register
    // copies per step).
    const int full_lim = CAUSAL ? min(qw0 - (BN - 1), S_kv - BN) : S_kv - BN;
    const int n_full = qw0 >= S_q ? 0 : min(nsteps, full_lim < 0 ? 0 : full_lim / BN + 1);
    // In these steps the copies of step + 1 go out once a sub-tile's S/dP
    // chains are issued, so that the wave's issue stall overlaps them
    // (issued right after the barrier, the copy burst of the four waves held
    // each of them ~560 clk per step): waves 0-1 after the first sub-tile's
    // chains, waves 2-3 after the second's, so that fewer copies queue in
    // the CU's address unit at once (1.6% faster at c4 than all four after
    // the first).  An L2 prefetch of the step after next (one dword per
    // line) made the kernel slower.
    int step = 0;
    for (; step < n_full; ++step) {
        wait_vm();
        __syncthreads();
        const uint32_t kbase = (uint32_t)((step & 1) * Cfg::STAGE);
        sub.template operator()<false>(kbase, step * BN, 0, [&] {
            if (step + 1 < nsteps && wave < 2) issue(step + 1);
        });
        sub.template operator()<false>(kbase, step * BN + 32, 1, [&] {
            if (step + 1 < nsteps && wave >= 2) issue(step + 1);
        });
    }
    for (; step < nsteps; ++step) {
        sync_step(step);
        if (qw0 >= S_q) continue;
        const int kv0 = step * BN;
        const uint32_t kbase = (uint32_t)((step & 1) * Cfg::STAGE);
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            const int k0 = kv0 + 32 * t;
            if (!(k0 < S_kv && (!CAUSAL || k0 <= qw0 + 31))) continue;
            sub.template operator()<true>(kbase, k0, t, none);
        }
    }

    if (row_ok) {
        half_t* dQb = static_cast<half_t*>(p.dq) + row_q * D_qk;
        if (D_qk == DQK) store_rows_f16<DQK>(dQb, dqacc, p.c.scale, hh);
        else store_rows_f16_n<DQK>(dQb, dqacc, p.c.scale, hh, D_qk);
    }
}


}  // namespace

hipError_t launch_bwd_dq_f16_dma(const BwdParams& p, hipStream_t stream) {
    const int B = p.s.B, S_q = p.s.S_q;
    if (B == 0 || S_q == 0) return hipSuccess;
    return with_dim(p.s.D_qk, [&](auto dqk) {
        return with_dim(p.s.D_v, [&](auto dv) {
            return with_bool(p.c.causal != 0, [&](auto c) {
                return with_bool(p.c.use_dropout != 0, [&](auto d) {
                    constexpr int DQK = decltype(dqk)::value, DV = decltype(dv)::value;
                    constexpr bool CA = decltype(c)::value, DR = decltype(d)::value;
                    using CQ = DqDmaCfg<DQK, DV>;
                    const long long n = (long long)((S_q + CQ::BM - 1) / CQ::BM) * B;
                    return launch_kernel<sdpa_bwd_dq_f16_dma_kernel<DQK, DV, CA, DR>>((unsigned)n, CQ::NT,
                                                                                CQ::LDS_BYTES, stream, p,
                                                                                row_window((size_t)p.s.S_kv * (DQK + DV) * 2));
                });
            });
        });
    });
}

}  // namespace sdpa
