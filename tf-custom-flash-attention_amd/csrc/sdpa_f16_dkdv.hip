// sdpa_f16_dkdv.hip -- fp16 SdpaGrad dK/dV kernels for gfx950 that stream
// their Q/dO tiles from HBM straight into LDS (the dQ kernel is in
// sdpa_f16_dq.hip, the forward in sdpa_f16_fwd.hip, the copy machinery in
// sdpa_dma.h), and the launcher of the fp16 DMA backward.
//
// These are the production dK/dV kernels for the fp16 op whenever every
// feature width is a multiple of 8 and every tensor is 16-byte aligned (the
// shapes the reference's MHA layer produces, sdpa_fwd.cu.cc:191-215 dispatch
// up to D = 128).  Other fp16 shapes use the register-staged kernels of
// sdpa_bwd.hip, which accept any D.
//
// The buffer descriptor of every tile starts at the tile's first row and ends
// at the end of the batch row, so rows past S and columns past D read as
// zero: tails need no branches.  Q/dO blocks pass through a ring of three LDS
// stages.
//
// Work order.  Workgroup ids are remapped so that each XCD (ids are dealt
// round-robin over the 8 XCDs) owns whole batch rows: all tiles of a batch
// row run on one XCD and share its L2 copy of the streamed operands; the
// tiles of a chunk of rows are interleaved (xcd_map, row_window).
//
// MFMA formulation (v_mfma_f32_32x32x16_f16, fp32 accumulation; the lane
// layouts are listed in sdpa_device.h), per group of 32 keys (lane = key):
//   S = Q K^T, dP = dO V^T, dV^T += dO^T P~, dK^T += Q^T dS
//   (one wave per group here; at a 128-wide side two, one for S, P and dV,
//   one for dP, dS and dK: sdpa_f16_dkdv_split.hip)
// Element semantics are those of the reference (sdpa/sdpa_bwd.cu.cc:130-170,
// 291-327), restated in sdpa_bwd.hip.
#include <type_traits>

#include "sdpa_dma.h"
#include "sdpa_launch.h"
#include "sdpa_params.h"

namespace sdpa {
namespace {

// ===========================================================================
// Backward, dK/dV kernel (reads stats2 and delta from the workspace)
// ===========================================================================
// Shapes with a 128-wide side run the split-role kernel
// (sdpa_f16_dkdv_split.hip) unless this is 0.
#ifndef SDPA_DKDV_SPLIT
#define SDPA_DKDV_SPLIT 1
#endif


template <int DQK, int DV>
struct DkvDmaCfg {
    static constexpr int NT = 256, BKV = 128, BQ = 64;
    static constexpr int LQ = DQK / 8, LO = DV / 8;
    static constexpr int QB = BQ * DQK * 2, OB = BQ * DV * 2, FB = 2 * BQ * 4;
    static constexpr int STAGE = QB + OB + FB;
    // waves per SIMD: with a 128-wide side, K, V, dK and dV of 32 keys plus
    // the step's working set do not fit in 256 VGPRs, so those shapes run one
    // wave per SIMD (one workgroup per CU, which leaves LDS for a deeper ring).
    static constexpr int WAVES = (DQK == 128 || DV == 128) ? 1 : 2;
    static constexpr int NSTAGE = (WAVES == 1 || 3 * STAGE <= 80 * 1024) ? 3 : 2;
    static constexpr size_t LDS_BYTES = NSTAGE * (size_t)STAGE;
};

template <int DQK, int DV, bool CAUSAL, bool DROP>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(DkvDmaCfg<DQK, DV>::WAVES, DkvDmaCfg<DQK, DV>::WAVES)))
void sdpa_bwd_dkdv_f16_dma_kernel(const BwdParams p, const int win) {
    using Cfg = DkvDmaCfg<DQK, DV>;
    constexpr int BKV = Cfg::BKV, BQ = Cfg::BQ, LQ = Cfg::LQ, LO = Cfg::LO;

    const int tid = threadIdx.x, lane = tid & 63, l32 = lane & 31, hh = lane >> 5;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int B = p.s.B, S_q = p.s.S_q, S_kv = p.s.S_kv, D_qk = p.s.D_qk, D_v = p.s.D_v;
    const int tiles = (S_kv + BKV - 1) / BKV;
    int b, kt;
    xcd_map(blockIdx.x, B * tiles, tiles, false, win, b, kt);
    const int k0 = kt * BKV, kw0 = k0 + 32 * wave, my_k = kw0 + l32;
    const bool key_ok = my_k < S_kv;

    const half_t* Qb = static_cast<const half_t*>(p.q) + (size_t)b * S_q * D_qk;
    const half_t* dOb = static_cast<const half_t*>(p.d_o) + (size_t)b * S_q * D_v;
    const half_t* Kb = static_cast<const half_t*>(p.k) + (size_t)b * S_kv * D_qk;
    const half_t* Vb = static_cast<const half_t*>(p.v) + (size_t)b * S_kv * D_v;
    const float* st2b = p.stats2 + (size_t)b * S_q;
    const float* deltab = p.delta + (size_t)b * S_q;

    // K and V rows of this lane's key as B operands.
    half8 kreg[DQK / 16], vreg[DV / 16];
#pragma unroll
    for (int ks = 0; ks < DQK / 16; ++ks)
        kreg[ks] = __builtin_bit_cast(half8, load_row_chunk<half_t, true>(Kb, my_k, S_kv, 16 * ks + 8 * hh, D_qk, D_qk));
#pragma unroll
    for (int ks = 0; ks < DV / 16; ++ks)
        vreg[ks] = __builtin_bit_cast(half8, load_row_chunk<half_t, true>(Vb, my_k, S_kv, 16 * ks + 8 * hh, D_v, D_v));
    prologue_loads_landed();

    // Queries below k0 see none of these keys under the causal mask.  The
    // query blocks are walked top-down: every key tile of a batch row starts
    // at the same (last) block and they move down together, so concurrent
    // workgroups read the same Q/dO rows while they are in L2.
    const int q_begin = CAUSAL ? (min(k0, S_q) / BQ) * BQ : 0;
    const int nsteps = (S_q - q_begin + BQ - 1) / BQ;
    const int q_top = q_begin + (nsteps - 1) * BQ;

    constexpr int NSTAGE = Cfg::NSTAGE;
    TileDma<BQ, LQ, 4> qd;
    TileDma<BQ, LO, 4> od;
    // copies issued by every wave per step (waves 0 and 1 add one each)
    constexpr int LPS = TileDma<BQ, LQ, 4>::MIN_PER_WAVE + TileDma<BQ, LO, 4>::MIN_PER_WAVE;
    qd.init(wave, lane, D_qk * 2, D_qk / 8);
    od.init(wave, lane, D_v * 2, D_v / 8);
    auto issue = [&](int step) {
        const int q0 = q_top - step * BQ;
        unsigned char* st = smem + (step % NSTAGE) * Cfg::STAGE;
        qd.issue(make_rsrc(Qb + (size_t)q0 * D_qk, (long long)(S_q - q0) * D_qk * 2), st, wave);
        od.issue(make_rsrc(dOb + (size_t)q0 * D_v, (long long)(S_q - q0) * D_v * 2), st + Cfg::QB, wave);
        if (wave == 0) dma4(make_rsrc(st2b + q0, (long long)(S_q - q0) * 4), st + Cfg::QB + Cfg::OB, lane * 4);
        if (wave == 1) dma4(make_rsrc(deltab + q0, (long long)(S_q - q0) * 4), st + Cfg::QB + Cfg::OB + BQ * 4, lane * 4);
    };
#pragma unroll
    for (int i = 0; i < NSTAGE - 1; ++i)
        if (i < nsteps) issue(i);
    // Wait for block `step` (the copies of the NSTAGE - 2 later blocks may
    // still fly; all of them at the tail) and synchronise.  The copy of block
    // step + NSTAGE - 1 goes out at the end of the step (`next_copy`), where
    // its issue stall overlaps the wave's wait at the following barrier; its
    // stage held block step - 1, which every wave finished before this
    // step's barrier (NSTAGE >= 3 keeps one step of prefetch).
    static_assert(NSTAGE >= 3 || Cfg::WAVES != 1, "end-of-step copies need a third stage");
    auto sync_step = [&](int step) {
        if (step + NSTAGE - 2 < nsteps) wait_vm_n<(NSTAGE - 2) * LPS>();
        else wait_vm();
        __syncthreads();
        if (NSTAGE < 3 && step + NSTAGE - 1 < nsteps) issue(step + NSTAGE - 1);
    };
    auto next_copy = [&](int step) {
        if (NSTAGE >= 3 && step + NSTAGE - 1 < nsteps) issue(step + NSTAGE - 1);
    };

    const float sl2 = p.c.scale_log2;
    const float ksc = p.c.keep_scale;
    // Dropout: st(q, key) = st(4 hh, key) + q * S_kv * A; the row step is uniform.
    const uint64_t st_lane = DROP ? lcg_state(p.c.seed_offset, (uint64_t)b * S_q + 4 * hh, (uint64_t)S_kv, my_k) : 0;
    const uint64_t row_step = (uint64_t)S_kv * kLcgMul;
    const uint32_t thr = p.c.drop_threshold;

    SwzLane<LQ> swQ;
    SwzLane<LO> swO;
    swQ.init(lane);
    swO.init(lane);

    floatx16 dkacc[DQK / 32], dvacc[DV / 32];
#pragma unroll
    for (int dt = 0; dt < DQK / 32; ++dt) dkacc[dt] = floatx16{};
#pragma unroll
    for (int dt = 0; dt < DV / 32; ++dt) dvacc[dt] = floatx16{};

    // Element-wise part of one 32-query sub-tile: the accumulator rows are
    // queries qs + 8 g + 4 hh + e; st4 / de4 hold their stats2
    // (stats log2(e) + kGateShift) and delta.  Produces the fp16 B operands
    // P~ (for dV) and dS (for dK).
    auto elem = [&]<bool MASK>(const floatx16& sacc, const floatx16& dpacc, const floatx4 (&st4)[4],
                               const floatx4 (&de4)[4], int qs, half8& pk0, half8& pk1, half8& ds0, half8& ds1) {
        const uint64_t st_sub = DROP ? st_lane + (uint64_t)qs * row_step : 0;
        uint32_t wp[8], wd[8];
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            float pk4[4], ds4[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int r = 4 * g + e;
                // stats2 carries kGateShift: exp2 gives P' (0 where P <= 1e-6)
                float x = __builtin_fmaf(sacc[r], sl2, -st4[g][e]);
                // masked: keys after the query (causal) and rows past S_q, whose
                // zero-filled stats2 would make P = 2^kGateShift
                if (MASK && ((CAUSAL && my_k > qs + 8 * g + 4 * hh + e) || qs + 8 * g + 4 * hh + e >= S_q))
                    x = -INFINITY;
                const float pr = fast_exp2(x) * kGateScale;
                if constexpr (DROP) {
                    const bool keep = lcg_keep(st_sub + (uint64_t)(8 * g + e) * row_step, thr);
                    pk4[e] = keep ? pr : 0.f;
                    ds4[e] = pr * (keep ? __builtin_fmaf(dpacc[r], ksc, -de4[g][e]) : -de4[g][e]);
                } else {
                    pk4[e] = pr;
                    ds4[e] = pr * (dpacc[r] - de4[g][e]);
                }
            }
            wp[2 * g] = pack_h2(pk4[0], pk4[1]);
            wp[2 * g + 1] = pack_h2(pk4[2], pk4[3]);
            wd[2 * g] = pack_h2(ds4[0], ds4[1]);
            wd[2 * g + 1] = pack_h2(ds4[2], ds4[3]);
        }
        pk0 = half8_of(wp[0], wp[1], wp[2], wp[3]);
        pk1 = half8_of(wp[4], wp[5], wp[6], wp[7]);
        ds0 = half8_of(wd[0], wd[1], wd[2], wd[3]);
        ds1 = half8_of(wd[4], wd[5], wd[6], wd[7]);
    };
    auto read_f = [&](const float* Fs, int t, floatx4 (&st4)[4], floatx4 (&de4)[4]) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            st4[g] = *reinterpret_cast<const floatx4*>(Fs + 32 * t + 8 * g + 4 * hh);
            de4[g] = *reinterpret_cast<const floatx4*>(Fs + BQ + 32 * t + 8 * g + 4 * hh);
        }
    };

    // One step of 64 queries whose two 32-query sub-tiles are fully visible
    // to the wave's keys, written in software-pipeline order (a wave issues
    // in order, so the element-wise work of one sub-tile is placed next to
    // the MFMAs of another; the compiler interleaves within each span):
    //   R1  A(0): S, dP of sub-tile 0           || reads of A(1) operands, F(0)
    //   R2  A(1)                                 || B(0) elementwise, reads of C(0) operands, F(1)
    //   R3  C(0): dV += dO0^T P0~, dK += Q0^T dS0 || B(1), reads of C(1) operands
    //   R4  C(1)
    constexpr int NK = DQK / 16, NV = DV / 16, NA = NK > NV ? NK : NV;
    auto full_step = [&](uint32_t qbase, int q0) {
        const uint32_t obase = qbase + Cfg::QB;
        const float* Fs = reinterpret_cast<const float*>(smem + obase + Cfg::OB);
        const uint32_t aQ = qbase + swQ.row, aO = obase + swO.row;
        const uint32_t aQ0 = qbase + swQ.tr0, aQ1 = qbase + swQ.tr1;
        const uint32_t aO0 = obase + swO.tr0, aO1 = obase + swO.tr1;
        half8 aq0[NK], ao0[NV], aq1[NK], ao1[NV];
#pragma unroll
        for (int ks = 0; ks < NA; ++ks) {
            if (ks < NK) aq0[ks] = lds_row<LQ>(aQ, ks, 0);
            if (ks < NV) ao0[ks] = lds_row<LO>(aO, ks, 0);
        }
        // ---- R1
        floatx16 s0 = floatx16{}, d0 = floatx16{}, s1 = floatx16{}, d1 = floatx16{};
#pragma unroll
        for (int ks = 0; ks < NA; ++ks) {
            if (ks < NK) s0 = mfma_f16(aq0[ks], kreg[ks], s0);
            if (ks < NV) d0 = mfma_f16(ao0[ks], vreg[ks], d0);
        }
#pragma unroll
        for (int ks = 0; ks < NA; ++ks) {
            if (ks < NK) aq1[ks] = lds_row<LQ>(aQ, ks, 32);
            if (ks < NV) ao1[ks] = lds_row<LO>(aO, ks, 32);
        }
        floatx4 f0s[4], f0d[4], f1s[4], f1d[4];
        read_f(Fs, 0, f0s, f0d);
        // ---- R2
#pragma unroll
        for (int ks = 0; ks < NA; ++ks) {
            if (ks < NK) s1 = mfma_f16(aq1[ks], kreg[ks], s1);
            if (ks < NV) d1 = mfma_f16(ao1[ks], vreg[ks], d1);
        }
        half8 cv0[2][DV / 32], cq0[2][DQK / 32], cv1[2][DV / 32], cq1[2][DQK / 32];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
#pragma unroll
            for (int dt = 0; dt < DV / 32; ++dt) cv0[j][dt] = lds_tr<LO>(aO0, aO1, dt, 16 * j);
#pragma unroll
            for (int dt = 0; dt < DQK / 32; ++dt) cq0[j][dt] = lds_tr<LQ>(aQ0, aQ1, dt, 16 * j);
        }
        read_f(Fs, 1, f1s, f1d);
        half8 pk00, pk01, ds00, ds01;
        elem.template operator()<false>(s0, d0, f0s, f0d, q0, pk00, pk01, ds00, ds01);
        // ---- R3
#pragma unroll
        for (int dt = 0; dt < DV / 32; ++dt) {
            dvacc[dt] = mfma_f16(cv0[0][dt], pk00, dvacc[dt]);
            dvacc[dt] = mfma_f16(cv0[1][dt], pk01, dvacc[dt]);
        }
#pragma unroll
        for (int dt = 0; dt < DQK / 32; ++dt) {
            dkacc[dt] = mfma_f16(cq0[0][dt], ds00, dkacc[dt]);
            dkacc[dt] = mfma_f16(cq0[1][dt], ds01, dkacc[dt]);
        }
#pragma unroll
        for (int j = 0; j < 2; ++j) {
#pragma unroll
            for (int dt = 0; dt < DV / 32; ++dt) cv1[j][dt] = lds_tr<LO>(aO0, aO1, dt, 32 + 16 * j);
#pragma unroll
            for (int dt = 0; dt < DQK / 32; ++dt) cq1[j][dt] = lds_tr<LQ>(aQ0, aQ1, dt, 32 + 16 * j);
        }
        half8 pk10, pk11, ds10, ds11;
        elem.template operator()<false>(s1, d1, f1s, f1d, q0 + 32, pk10, pk11, ds10, ds11);
        // ---- R4
#pragma unroll
        for (int dt = 0; dt < DV / 32; ++dt) {
            dvacc[dt] = mfma_f16(cv1[0][dt], pk10, dvacc[dt]);
            dvacc[dt] = mfma_f16(cv1[1][dt], pk11, dvacc[dt]);
        }
#pragma unroll
        for (int dt = 0; dt < DQK / 32; ++dt) {
            dkacc[dt] = mfma_f16(cq1[0][dt], ds10, dkacc[dt]);
            dkacc[dt] = mfma_f16(cq1[1][dt], ds11, dkacc[dt]);
        }
    };

    // One 32-query sub-tile that needs the causal mask (or lies past it),
    // computed without pipelining: qs = first query, t = 0 / 1 within the step.
    auto masked_sub = [&]<bool PART>(uint32_t qbase, int t, int qs) __attribute__((always_inline)) {
        const uint32_t obase = qbase + Cfg::QB;
        const float* Fs = reinterpret_cast<const float*>(smem + obase + Cfg::OB);
        const uint32_t aQ = qbase + swQ.row, aO = obase + swO.row;
        const uint32_t aQ0 = qbase + swQ.tr0, aQ1 = qbase + swQ.tr1;
        const uint32_t aO0 = obase + swO.tr0, aO1 = obase + swO.tr1;
        floatx16 sacc = floatx16{}, dpacc = floatx16{};
#pragma unroll
        for (int ks = 0; ks < NK; ++ks) sacc = mfma_f16(lds_row<LQ>(aQ, ks, 32 * t), kreg[ks], sacc);
#pragma unroll
        for (int ks = 0; ks < NV; ++ks) dpacc = mfma_f16(lds_row<LO>(aO, ks, 32 * t), vreg[ks], dpacc);
        floatx4 fs[4], fd[4];
        read_f(Fs, t, fs, fd);
        half8 pk0, pk1, ds0, ds1;
        elem.template operator()<PART>(sacc, dpacc, fs, fd, qs, pk0, pk1, ds0, ds1);
#pragma unroll
        for (int dt = 0; dt < DV / 32; ++dt) {
            dvacc[dt] = mfma_f16(lds_tr<LO>(aO0, aO1, dt, 32 * t), pk0, dvacc[dt]);
            dvacc[dt] = mfma_f16(lds_tr<LO>(aO0, aO1, dt, 32 * t + 16), pk1, dvacc[dt]);
        }
#pragma unroll
        for (int dt = 0; dt < DQK / 32; ++dt) {
            dkacc[dt] = mfma_f16(lds_tr<LQ>(aQ0, aQ1, dt, 32 * t), ds0, dkacc[dt]);
            dkacc[dt] = mfma_f16(lds_tr<LQ>(aQ0, aQ1, dt, 32 * t + 16), ds1, dkacc[dt]);
        }
    };

    // Steps whose 64 queries all see all 32 keys of the wave come first
    // (top-down walk); the causal diagonal and the blocks below it follow.
    // Only the one-wave-per-SIMD shape has the registers for the pipelined
    // step; the others run the full steps as two plain sub-tiles, in a loop
    // of their own: one loop over every kind of step merged the dK/dV
    // accumulators of its paths with 32 register copies per sub-tile.
    // The top block takes the full path only when it lies entirely below S_q.
    const int n_full = kw0 >= S_kv ? 0
                       : !CAUSAL   ? nsteps
                                   : (q_top >= kw0 + 32 ? min(nsteps, (q_top - kw0 - 32) / BQ + 1) : 0);
    int step = 0;
    auto masked_step = [&](int step) {
        sync_step(step);
        if (kw0 < S_kv) {
            const int q0 = q_top - step * BQ;
            const uint32_t qbase = (uint32_t)((step % NSTAGE) * Cfg::STAGE);
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                const int qs = q0 + 32 * t;
                if (qs >= S_q || (CAUSAL && qs + 31 < kw0)) continue;
                // every live sub-tile takes the masked path: with the
                // unmasked one as well, the loop merged the dK/dV
                // accumulators of the two with 64 register copies per step
                masked_sub.template operator()<true>(qbase, t, qs);
            }
        }
        next_copy(step);
    };
    if (n_full > 0 && q_top + BQ > S_q) masked_step(step++);
    if constexpr (Cfg::WAVES != 1) {
        for (; step < n_full; ++step) {
            sync_step(step);
            const int q0 = q_top - step * BQ;
            const uint32_t qbase = (uint32_t)((step % NSTAGE) * Cfg::STAGE);
            masked_sub.template operator()<false>(qbase, 0, q0);
            masked_sub.template operator()<false>(qbase, 1, q0 + 32);
            next_copy(step);
        }
    } else {
        for (; step < n_full; ++step) {
            sync_step(step);
            full_step((uint32_t)((step % NSTAGE) * Cfg::STAGE), q_top - step * BQ);
            next_copy(step);
        }
    }
    for (; step < nsteps; ++step) masked_step(step);

    if (key_ok) {
        half_t* dKb = static_cast<half_t*>(p.dk) + ((size_t)b * S_kv + my_k) * D_qk;
        half_t* dVb = static_cast<half_t*>(p.dv) + ((size_t)b * S_kv + my_k) * D_v;
        if (D_qk == DQK) store_rows_f16<DQK>(dKb, dkacc, p.c.scale, hh);
        else store_rows_f16_n<DQK>(dKb, dkacc, p.c.scale, hh, D_qk);
        if (D_v == DV) store_rows_f16<DV>(dVb, dvacc, p.c.keep_scale, hh);
        else store_rows_f16_n<DV>(dVb, dvacc, p.c.keep_scale, hh, D_v);
    }
}

}  // namespace

// ---------------------------------------------------------------------------
// Host launchers
// ---------------------------------------------------------------------------
hipError_t launch_bwd_f16_dma(const BwdParams& p, int phases, hipStream_t stream) {
    const int B = p.s.B, S_q = p.s.S_q, S_kv = p.s.S_kv;
    if (B == 0) return hipSuccess;
    return with_dim(p.s.D_qk, [&](auto dqk) {
        return with_dim(p.s.D_v, [&](auto dv) {
            return with_bool(p.c.causal != 0, [&](auto c) {
                return with_bool(p.c.use_dropout != 0, [&](auto d) {
                    constexpr int DQK = decltype(dqk)::value, DV = decltype(dv)::value;
                    constexpr bool CA = decltype(c)::value, DR = decltype(d)::value;
                    using CK = DkvDmaCfg<DQK, DV>;
                    hipError_t err = hipSuccess;
                    if ((phases & kBwdDq) && S_q > 0) err = launch_bwd_dq_f16_dma(p, stream);
                    if (err == hipSuccess && (phases & kBwdDkDv) && S_kv > 0) {
                        if constexpr (CK::WAVES == 1 && SDPA_DKDV_SPLIT) {
                            err = launch_bwd_dkdv_f16_split(p, stream);
                        } else {
                            const long long n = (long long)((S_kv + CK::BKV - 1) / CK::BKV) * B;
                            err = launch_kernel<sdpa_bwd_dkdv_f16_dma_kernel<DQK, DV, CA, DR>>(
                                (unsigned)n, CK::NT, CK::LDS_BYTES, stream, p,
                                row_window((size_t)S_q * (DQK + DV) * 2));
                        }
                    }
                    return err;
                });
            });
        });
    });
}

}  // namespace sdpa
