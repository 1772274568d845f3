// sdpa_f16_dkdv_split.hip -- fp16 SdpaGrad dK/dV kernel for gfx950 at a
// 128-wide feature side (D_qk or D_v = 128): the work of each group of 32
// keys split over two waves (S, P and dV; dP, dS and dK), Q/dO tiles
// streamed from HBM straight into LDS (copy machinery in sdpa_dma.h).  The
// one-wave kernel for D <= 64 and the launcher of the fp16 DMA backward are
// in sdpa_f16_dkdv.hip.
//
// A file of its own so that it can be built with LLVM's max-ilp machine
// scheduler: c4's dK/dV 1.39 against 1.41 ms, without dropout 1.28 against
// 1.36 ms, bit-identical (the one-wave kernel is 10% slower with it).
//
// Element semantics are those of the reference (sdpa/sdpa_bwd.cu.cc:130-170,
// 291-327), restated in sdpa_bwd.hip.
#include <type_traits>

#include "sdpa_dma.h"
#include "sdpa_launch.h"
#include "sdpa_params.h"

// Split-role kernel, who copies the tiles: 0 the dS role; 1 the P role under
// the causal mask, else the dS role; 2 the P role.
#ifndef SDPA_DKDV_PCOPY
#define SDPA_DKDV_PCOPY 1
#endif

namespace sdpa {
namespace {

// The P role hands P to the dS role (and into its own dV product) as fp16
// x = P 2^kXShift: P ranges over [1e-6, 1] (the gate below, the row
// statistics above), and 2^6 puts all of it in fp16's normal range.
constexpr float kXScale = 64.f;  // 2^kXShift, kXShift = 6

// ===========================================================================
// Backward, dK/dV kernel with the work of a key split over two waves
// ===========================================================================
// Eight waves over 128 keys.  Waves w and w + 4 (w < 4) own keys
// k0 + 32 w .. + 31 and run on the same SIMD:
//   wave w      (P role):  S = Q K^T, P = exp2(S sl2 - stats2) 2^kGateShift
//                          (stats2 carries the shift; see kGateShift), P~ = P * keep,
//                          dV^T += dO^T P~; it hands P to wave w + 4 through
//                          LDS with the dropout decision in the sign (-P for a
//                          dropped element), as fp16 P 2^kXShift (kXScale);
//   wave w + 4  (dS role): dP = dO V^T, dS = P (keep ? dP ksc - delta : -delta),
//                          dK^T += Q^T dS, one block behind the P role.
// Each role holds one operand (K or V, 32 VGPRs) and one accumulator (64), so
// both roles fit two waves per SIMD, and every SIMD still does the four GEMMs
// of its 32 keys once per block.  The tiles are copied by the P role under
// the causal mask (it issues them right after its S chains, in time it would
// otherwise spend waiting at the barrier for the dS role) and by the dS role
// otherwise (there the P role has no registers to spare for the copy state).
//
// LDS: a ring of three blocks (Q, dO, stats2, delta) and two P exchange
// buffers.  During step n the P role reads block n, the dS role reads block
// n - 1 and P of step n - 1, and the copy of block n + 1 is in flight; it was
// issued after the barrier that opened step n, into the ring slot of block
// n - 2.
template <int DQK, int DV>
struct DkvSplitCfg {
    static constexpr int NT = 512, BKV = 128, BQ = 64, NSTAGE = 3;
    static constexpr int LQ = DQK / 8, LO = DV / 8;
    static constexpr int QB = BQ * DQK * 2, OB = BQ * DV * 2, FB = 2 * BQ * 4;
    static constexpr int STAGE = QB + OB + FB;
    // P of one block: 4 key groups x 2 sub-tiles x 64 lanes x 16 halves
    static constexpr int XB = 4 * 2 * 64 * 32;
    static constexpr size_t LDS_BYTES = NSTAGE * (size_t)STAGE + 2 * XB;
    static_assert(LDS_BYTES <= 160 * 1024, "gfx950 LDS");
};

template <int DQK, int DV, bool CAUSAL, bool DROP, bool DS>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
void sdpa_bwd_dkdv_f16_split_kernel(const BwdParams p, const int win) {
    using Cfg = DkvSplitCfg<DQK, DV>;
    constexpr bool PCOPY = SDPA_DKDV_PCOPY == 2 || (SDPA_DKDV_PCOPY == 1 && CAUSAL);
    constexpr int BKV = Cfg::BKV, BQ = Cfg::BQ, LQ = Cfg::LQ, LO = Cfg::LO, NSTAGE = Cfg::NSTAGE;

    const int tid = threadIdx.x, lane = tid & 63, l32 = lane & 31, hh = lane >> 5;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int kw = wave & 3;
    const int B = p.s.B, S_q = p.s.S_q, S_kv = p.s.S_kv, D_qk = p.s.D_qk, D_v = p.s.D_v;
    const int tiles = (S_kv + BKV - 1) / BKV;
    int b, kt;
    xcd_map(blockIdx.x, B * tiles, tiles, false, win, b, kt);
    const int k0 = kt * BKV, kw0 = k0 + 32 * kw, my_k = kw0 + l32;
    const bool key_ok = my_k < S_kv;

    const half_t* Qb = static_cast<const half_t*>(p.q) + (size_t)b * S_q * D_qk;
    const half_t* dOb = static_cast<const half_t*>(p.d_o) + (size_t)b * S_q * D_v;

    // Query blocks walked top-down (see the one-wave kernel above).
    const int q_begin = CAUSAL ? (min(k0, S_q) / BQ) * BQ : 0;
    const int nsteps = (S_q - q_begin + BQ - 1) / BQ;
    const int q_top = q_begin + (nsteps - 1) * BQ;

    // Sub-tile t of block m: queries qs = q0 + 32 t; skipped (by both roles)
    // when past S_q, past the keys or, under the causal mask, above every key.
    auto sub_live = [&](int qs) {
        return kw0 < S_kv && qs < S_q && !(CAUSAL && qs + 31 < kw0);
    };
    auto xbuf = [&](int m, int t) {
        return smem + NSTAGE * Cfg::STAGE + (m & 1) * Cfg::XB + (kw * 2 + t) * 2048 + lane * 16;
    };

    if (wave < 4) {
        // ------------------------------------------------------------ P role
        half8 kreg[DQK / 16];
        const half_t* Kb = static_cast<const half_t*>(p.k) + (size_t)b * S_kv * D_qk;
#pragma unroll
        for (int ks = 0; ks < DQK / 16; ++ks)
            kreg[ks] = __builtin_bit_cast(half8, load_row_chunk<half_t, true>(Kb, my_k, S_kv, 16 * ks + 8 * hh, D_qk, D_qk));
        prologue_loads_landed();
        const float sl2 = p.c.scale_log2;
        // Dropout: st(q, key) = st(4 hh, key) + q * S_kv * A.
        const uint64_t st_lane = DROP ? lcg_state(p.c.seed_offset, (uint64_t)b * S_q + 4 * hh, (uint64_t)S_kv, my_k) : 0;
        const uint64_t row_step = (uint64_t)S_kv * kLcgMul;
        const uint32_t thr = p.c.drop_threshold;
        SwzLane<LQ> swQ;
        SwzLane<LO> swO;
        swQ.init(lane);
        swO.init(lane);
        // Tile copies (PCOPY).  Block m + 1 goes out while this role works on block m,
        // right after its S chains: its stage held block m - 2, which the dS
        // role released at barrier m, and it lands before barrier m + 1.  The
        // dS role, which issued them before, has no time to spare: this
        // role waited at the barrier for it (the dS role's tail, or the copies
        // split between the roles, measured slower).  With dropout the delta
        // row of each block is then rewritten as delta' (see the dS role) by
        // the wave that copied it.
        const float* st2b = p.stats2 + (size_t)b * S_q;
        const float* deltab = p.delta + (size_t)b * S_q;
        TileDma<BQ, LQ, 4> qd;
        TileDma<BQ, LO, 4> od;
        qd.init(kw, lane, D_qk * 2, D_qk / 8);
        od.init(kw, lane, D_v * 2, D_v / 8);
        auto issue_block = [&](int m) {
            if (PCOPY && m < nsteps) {
                const int q0 = q_top - m * BQ;
                unsigned char* st = smem + (m % NSTAGE) * Cfg::STAGE;
                qd.issue(make_rsrc(Qb + (size_t)q0 * D_qk, (long long)(S_q - q0) * D_qk * 2), st, kw);
                od.issue(make_rsrc(dOb + (size_t)q0 * D_v, (long long)(S_q - q0) * D_v * 2), st + Cfg::QB, kw);
                if (kw == 0) dma4(make_rsrc(st2b + q0, (long long)(S_q - q0) * 4), st + Cfg::QB + Cfg::OB, lane * 4);
                if (kw == 1) dma4(make_rsrc(deltab + q0, (long long)(S_q - q0) * 4), st + Cfg::QB + Cfg::OB + BQ * 4, lane * 4);
            }
        };
        auto land_block = [&](int m) {
            if (PCOPY && m < nsteps) {
                wait_vm();
                if (DROP && kw == 1 && p.c.keep_scale != 0.f) {
                    float* dl = reinterpret_cast<float*>(smem + (m % NSTAGE) * Cfg::STAGE + Cfg::QB + Cfg::OB) + BQ;
                    dl[lane] = dl[lane] / p.c.keep_scale;
                }
            }
        };
        issue_block(0);
        land_block(0);
        floatx16 dvacc[DV / 32];
#pragma unroll
        for (int dt = 0; dt < DV / 32; ++dt) dvacc[dt] = floatx16{};

        // P of one sub-tile: xv = P with the dropout decision in the sign (for
        // the dS role), pk = max(xv, 0) = P~ (the dV B operand).
        auto elem = [&]<bool MASK>(const floatx16& sacc, const floatx4 (&st4)[4], int qs, half8& pk0, half8& pk1,
                                   half8& xv0, half8& xv1) {
            uint64_t st_sub = DROP ? st_lane + (uint64_t)qs * row_step : 0;
            // Hash states after S: computed all at once above the MFMAs they
            // would hold 32 VGPRs through the chain.
            if constexpr (DROP) asm volatile("" : "+v"(st_sub) : "v"(sacc[15]));
            // masked: query qs + 8 g + 4 hh + e is before key my_k (causal) iff
            // my_k - qs - 4 hh > 8 g + e, and past S_q iff 8 g + e >= S_q - qs - 4 hh
            // (its zero-filled stats2 would make P = 2^kGateShift); one lane
            // term each, against immediate bounds
            const int kd = MASK ? my_k - qs - 4 * hh : 0;
            const int qd = MASK ? S_q - qs - 4 * hh : 0;
            uint32_t wx[8];
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                float x4[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    float x = __builtin_fmaf(sacc[4 * g + e], sl2, -st4[g][e]);
                    if (MASK && ((CAUSAL && kd > 8 * g + e) || 8 * g + e >= qd)) x = -INFINITY;
                    // stats2 carries kGateShift: exp2 gives P' (0 where P <= 1e-6);
                    // x = P 2^kXShift keeps every P above the gate in fp16's
                    // normal range (2^-11 relative, not a subnormal's spacing)
                    const float pe = fast_exp2(x) * (kGateScale * kXScale);
                    if constexpr (DROP)
                        x4[e] = lcg_keep(st_sub + (uint64_t)(8 * g + e) * row_step, thr) ? pe : -pe;
                    else
                        x4[e] = pe;
                }
                wx[2 * g] = pack_h2(x4[0], x4[1]);
                wx[2 * g + 1] = pack_h2(x4[2], x4[3]);
            }
            xv0 = half8_of(wx[0], wx[1], wx[2], wx[3]);
            xv1 = half8_of(wx[4], wx[5], wx[6], wx[7]);
            if constexpr (DROP) {
                pk0 = relu_h8(xv0);
                pk1 = relu_h8(xv1);
            } else {
                pk0 = xv0;
                pk1 = xv1;
            }
        };
        auto sub = [&]<bool MASK>(uint32_t qbase, int m, int t, int qs) {
            const uint32_t obase = qbase + Cfg::QB;
            const float* Fs = reinterpret_cast<const float*>(smem + obase + Cfg::OB);
            const uint32_t aQ = qbase + swQ.row;
            const uint32_t aO0 = obase + swO.tr0, aO1 = obase + swO.tr1;
            floatx16 sacc = floatx16{};
#pragma unroll
            for (int ks = 0; ks < DQK / 16; ++ks) sacc = mfma_f16(lds_row<LQ>(aQ, ks, 32 * t), kreg[ks], sacc);
            floatx4 st4[4];
#pragma unroll
            for (int g = 0; g < 4; ++g) st4[g] = *reinterpret_cast<const floatx4*>(Fs + 32 * t + 8 * g + 4 * hh);
            half8 pk0, pk1, xv0, xv1;
            elem.template operator()<MASK>(sacc, st4, qs, pk0, pk1, xv0, xv1);
            unsigned char* xs = xbuf(m, t);
            *reinterpret_cast<half8*>(xs) = xv0;
            *reinterpret_cast<half8*>(xs + 1024) = xv1;
#pragma unroll
            for (int dt = 0; dt < DV / 32; ++dt) {
                dvacc[dt] = mfma_f16(lds_tr<LO>(aO0, aO1, dt, 32 * t), pk0, dvacc[dt]);
                dvacc[dt] = mfma_f16(lds_tr<LO>(aO0, aO1, dt, 32 * t + 16), pk1, dvacc[dt]);
            }
        };
        // A block whose two sub-tiles are both live and unmasked, in one
        // straight-line region: both S chains first, then each sub-tile's P
        // and dV.  The P work of sub-tile 0 then runs beside the S(1) MFMAs
        // and that of sub-tile 1 beside dV(0).  Sub-tile by sub-tile, a P
        // wave and its dS partner, released by the same barrier, started
        // every block with an MFMA burst and then both ran VALU work
        // (3% slower).
        // after_s runs once both S chains are issued, after_e0 once the
        // first sub-tile's P is written (the tile copies: a wave's issue
        // stall behind the CU's copy queue then overlaps work already in
        // flight; one wave's copies spread over the block stalled its
        // element-wise work instead, 4% slower).
        auto full = [&](uint32_t qbase, int m, int q0, auto&& after_s, auto&& after_e0) {
            const uint32_t obase = qbase + Cfg::QB;
            const float* Fs = reinterpret_cast<const float*>(smem + obase + Cfg::OB);
            const uint32_t aQ = qbase + swQ.row;
            const uint32_t aO0 = obase + swO.tr0, aO1 = obase + swO.tr1;
            floatx16 sacc[2] = {floatx16{}, floatx16{}};
#pragma unroll
            for (int t = 0; t < 2; ++t)
#pragma unroll
                for (int ks = 0; ks < DQK / 16; ++ks)
                    sacc[t] = mfma_f16(lds_row<LQ>(aQ, ks, 32 * t), kreg[ks], sacc[t]);
            __builtin_amdgcn_sched_barrier(0);
            after_s();
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                floatx4 st4[4];
#pragma unroll
                for (int g = 0; g < 4; ++g) st4[g] = *reinterpret_cast<const floatx4*>(Fs + 32 * t + 8 * g + 4 * hh);
                // The dV operands go out before the element-wise work and land
                // during it (read just before each MFMA, every MFMA waited
                // out the LDS latency: 2.5% slower).
                half8 at[2][DV / 32];
#pragma unroll
                for (int j = 0; j < 2; ++j)
#pragma unroll
                    for (int dt = 0; dt < DV / 32; ++dt) at[j][dt] = lds_tr<LO>(aO0, aO1, dt, 32 * t + 16 * j);
                __builtin_amdgcn_sched_barrier(0);
                half8 pk0, pk1, xv0, xv1;
                elem.template operator()<false>(sacc[t], st4, q0 + 32 * t, pk0, pk1, xv0, xv1);
                unsigned char* xs = xbuf(m, t);
                *reinterpret_cast<half8*>(xs) = xv0;
                *reinterpret_cast<half8*>(xs + 1024) = xv1;
                if (t == 0) {
                    __builtin_amdgcn_sched_barrier(0);
                    after_e0();
                    __builtin_amdgcn_sched_barrier(0);
                }
#pragma unroll
                for (int dt = 0; dt < DV / 32; ++dt) {
                    dvacc[dt] = mfma_f16(at[0][dt], pk0, dvacc[dt]);
                    dvacc[dt] = mfma_f16(at[1][dt], pk1, dvacc[dt]);
                }
            }
        };
        auto general = [&](int n) {
            const int q0 = q_top - n * BQ;
            const uint32_t qbase = (uint32_t)((n % NSTAGE) * Cfg::STAGE);
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                const int qs = q0 + 32 * t;
                // the masked path for every live sub-tile (see the dV note below)
                if (sub_live(qs)) sub.template operator()<true>(qbase, n, t, qs);
            }
        };
        // The blocks that take `full` form one run [n0, n1): only the top
        // block can reach past S_q (it then takes the masked path) and, causal,
        // the blocks past the first one that reaches the diagonal are
        // masked.  The run has a loop of its own, so that the dV
        // accumulators it carries stay in place (one loop over every kind of
        // block merged them from the three paths with 64 register copies per
        // block; the loops around it run the masked path only, for the same
        // reason).  nsteps + 1 barriers, as many as the dS role.
        int n0 = nsteps, n1 = nsteps;
        if (kw0 < S_kv) {
            n0 = (q_top + BQ <= S_q) ? 0 : 1;
            // full iff !(CAUSAL && q0 < kw0 + 31), q0 = q_top - 64 n
            n1 = CAUSAL ? (q_top >= kw0 + 31 ? min(nsteps, (q_top - (kw0 + 31)) / BQ + 1) : 0) : nsteps;
            n0 = min(n0, n1);
        }
        int n = 0;
        for (; n < n0; ++n) {
            __syncthreads();
            general(n);
            issue_block(n + 1);
            land_block(n + 1);
        }
        for (; n < n1; ++n) {
            __syncthreads();
            // Waves 0-1 issue their copies after the S chains, waves 2-3
            // after the first sub-tile's P: issued by all four at once, each
            // wave's copies queued behind the others' in the CU's address
            // unit (≈720 clk of issue stall per block; staggered, c4 dK/dV
            // 0.5-1.5% faster; a third point after dV(0) gained nothing).
            full((uint32_t)((n % NSTAGE) * Cfg::STAGE), n, q_top - n * BQ,
                 [&] { if (kw < 2) issue_block(n + 1); },
                 [&] { if (kw >= 2) issue_block(n + 1); });
            land_block(n + 1);
        }
        for (; n < nsteps; ++n) {
            __syncthreads();
            general(n);
            issue_block(n + 1);
            land_block(n + 1);
        }
        __syncthreads();
        if (key_ok) {
            half_t* dVb = static_cast<half_t*>(p.dv) + ((size_t)b * S_kv + my_k) * D_v;
            // dV was accumulated from x = P~ 2^kXShift
            const float fv = p.c.keep_scale * (1.f / kXScale);
            if (D_v == DV) store_rows_f16<DV>(dVb, dvacc, fv, hh);
            else store_rows_f16_n<DV>(dVb, dvacc, fv, hh, D_v);
        }
    } else {
        // ----------------------------------------------------------- dS role
        half8 vreg[DV / 16];
        const half_t* Vb = static_cast<const half_t*>(p.v) + (size_t)b * S_kv * D_v;
#pragma unroll
        for (int ks = 0; ks < DV / 16; ++ks)
            vreg[ks] = __builtin_bit_cast(half8, load_row_chunk<half_t, true>(Vb, my_k, S_kv, 16 * ks + 8 * hh, D_v, D_v));
        prologue_loads_landed();
        // With dropout the factor 1/(1-p) is taken out of dS: this role forms
        //   dS' = P (keep ? dP - delta' : -delta'),  delta' = delta / (1/(1-p))
        // (the reference's D_i / dp_inverse_scale, sdpa/sdpa_cpu.cc:428) and
        // dK is stored with scale / (1-p).  Each block's delta row is
        // rewritten as delta' in LDS once, by the wave that copies it.
        const float ksc = p.c.keep_scale;
        // keep_scale = 0 (dropout > 1: every element dropped in the reference,
        // dS = -P delta): dP is formed from zero V rows, delta is not rescaled
        // and dK is stored with scale, so dS' = -|x| delta for every element.
        const bool drop_all = DROP && ksc == 0.f;
        if (drop_all) {
#pragma unroll
            for (int ks = 0; ks < DV / 16; ++ks) vreg[ks] = half8{};
        }
        const float* st2b = p.stats2 + (size_t)b * S_q;
        const float* deltab = p.delta + (size_t)b * S_q;
        TileDma<BQ, LQ, 4> qd;
        TileDma<BQ, LO, 4> od;
        constexpr int LPS = TileDma<BQ, LQ, 4>::MIN_PER_WAVE + TileDma<BQ, LO, 4>::MIN_PER_WAVE;
        qd.init(kw, lane, D_qk * 2, D_qk / 8);
        od.init(kw, lane, D_v * 2, D_v / 8);
        auto issue = [&](int m) {
            const int q0 = q_top - m * BQ;
            unsigned char* st = smem + (m % NSTAGE) * Cfg::STAGE;
            qd.issue(make_rsrc(Qb + (size_t)q0 * D_qk, (long long)(S_q - q0) * D_qk * 2), st, kw);
            od.issue(make_rsrc(dOb + (size_t)q0 * D_v, (long long)(S_q - q0) * D_v * 2), st + Cfg::QB, kw);
            if (kw == 0) dma4(make_rsrc(st2b + q0, (long long)(S_q - q0) * 4), st + Cfg::QB + Cfg::OB, lane * 4);
            if (kw == 1) dma4(make_rsrc(deltab + q0, (long long)(S_q - q0) * 4), st + Cfg::QB + Cfg::OB + BQ * 4, lane * 4);
        };
        if (!PCOPY && nsteps > 0) issue(0);
        if (!PCOPY && nsteps > 1) issue(1);
        SwzLane<LQ> swQ;
        SwzLane<LO> swO;
        swQ.init(lane);
        swO.init(lane);
        floatx16 dkacc[DQK / 32];
#pragma unroll
        for (int dt = 0; dt < DQK / 32; ++dt) dkacc[dt] = floatx16{};
        const DsLayout dsl(S_q, S_kv, CAUSAL);

        // dS' of one sub-tile from dP, delta' and the P role's x.
        auto elem = [&](const floatx16& dpacc, const floatx4 (&de4)[4], const half8& xv0, const half8& xv1,
                        half8& ds0, half8& ds1) {
            // dS' = P (keep ? dP - delta' : -delta') = max(x, 0) dP - |x| delta'
            // (x 2^-kXShift: exact)
            uint32_t wd[8];
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                float ds4[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int r = 4 * g + e;
                    const float xq = (float)(r < 8 ? xv0[r] : xv1[r - 8]) * (1.f / kXScale);
                    const float mq = DROP ? fmaxf(xq, 0.f) : xq;
                    if constexpr (DROP)
                        ds4[e] = __builtin_fmaf(-__builtin_fabsf(xq), de4[g][e], mq * dpacc[r]);
                    else
                        ds4[e] = xq * (dpacc[r] - de4[g][e]);
                }
                wd[2 * g] = pack_h2(ds4[0], ds4[1]);
                wd[2 * g + 1] = pack_h2(ds4[2], ds4[3]);
            }
            ds0 = half8_of(wd[0], wd[1], wd[2], wd[3]);
            ds1 = half8_of(wd[4], wd[5], wd[6], wd[7]);
        };
        // one sub-tile: dP, dS' (returned in d0 / d1 for the dS store) and dK
        auto sub = [&](uint32_t qbase, int m, int t, half8& d0, half8& d1) {
            const uint32_t obase = qbase + Cfg::QB;
            const float* Fs = reinterpret_cast<const float*>(smem + obase + Cfg::OB);
            const uint32_t aO = obase + swO.row;
            const uint32_t aQ0 = qbase + swQ.tr0, aQ1 = qbase + swQ.tr1;
            floatx16 dpacc = floatx16{};
#pragma unroll
            for (int ks = 0; ks < DV / 16; ++ks) dpacc = mfma_f16(lds_row<LO>(aO, ks, 32 * t), vreg[ks], dpacc);
            floatx4 de4[4];
#pragma unroll
            for (int g = 0; g < 4; ++g) de4[g] = *reinterpret_cast<const floatx4*>(Fs + BQ + 32 * t + 8 * g + 4 * hh);
            const unsigned char* xs = xbuf(m, t);
            const half8 xv0 = *reinterpret_cast<const half8*>(xs), xv1 = *reinterpret_cast<const half8*>(xs + 1024);
            // the dK operands land during the element-wise work, as in the P role
            half8 at[2][DQK / 32];
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int dt = 0; dt < DQK / 32; ++dt) at[j][dt] = lds_tr<LQ>(aQ0, aQ1, dt, 32 * t + 16 * j);
            __builtin_amdgcn_sched_barrier(0);
            half8 ds0, ds1;
            elem(dpacc, de4, xv0, xv1, ds0, ds1);
            d0 = ds0;
            d1 = ds1;
#pragma unroll
            for (int dt = 0; dt < DQK / 32; ++dt) {
                dkacc[dt] = mfma_f16(at[0][dt], ds0, dkacc[dt]);
                dkacc[dt] = mfma_f16(at[1][dt], ds1, dkacc[dt]);
            }
        };
        // dS' of sub-tile t of block m into its chunk (DsLayout): store j of
        // this lane to slot(key, 2 j + h) of its key group, each store 1 KB in
        // runs of four lanes (key rows of 64 bytes, one 16-byte piece per lane,
        // made every lane a write request of its own); zero for keys past S_kv
        // (the dQ kernel reads them unmasked).  Both sub-tiles' dS'
        // go out at the end of the block, while the P role runs its dV
        // products rather than its copies (issued beside those copies they
        // cost c4's dK/dV 2.7% more), and non-temporal: the lines are not read
        // again here, and left in L2 they evict the Q / dO tiles this kernel
        // re-reads (a step 2.766 -> 2.720 ms; system-scope write-through 3.2 ms).
        auto store_ds = [&](int m, int t, half8 d0, half8 d1) {
            if (kw0 + 31 >= S_kv && !key_ok) {
                d0 = half8{};
                d1 = half8{};
            }
            const int qb = (q_top - m * BQ) / BQ;
            unsigned char* dst = static_cast<unsigned char*>(p.ds) + dsl.offset(b, kt, qb) + t * 8192 +
                                 kw * 2048;
            __builtin_nontemporal_store(d0, reinterpret_cast<half8*>(dst + DsLayout::slot(l32, hh)));
            __builtin_nontemporal_store(d1, reinterpret_cast<half8*>(dst + DsLayout::slot(l32, 2 + hh)));
        };
        if constexpr (PCOPY) {
        // The P role copies every block and rewrites its delta row before the
        // barrier that releases it: this role only multiplies.  nsteps + 1
        // barriers, as many as the P role: barrier n releases block n - 1 to
        // this role.
        __syncthreads();
        for (int n = 1; n <= nsteps; ++n) {
            __syncthreads();
            const int m = n - 1;
            const int q0 = q_top - m * BQ;
            const uint32_t qbase = (uint32_t)((m % NSTAGE) * Cfg::STAGE);
            half8 a0, a1, c0, c1;
            const bool l0 = sub_live(q0), l1 = sub_live(q0 + 32);
            if (l0) sub(qbase, m, 0, a0, a1);
            if (l1) sub(qbase, m, 1, c0, c1);
            if constexpr (DS) {
                if (l0) store_ds(m, 0, a0, a1);
                if (l1) store_ds(m, 1, c0, c1);
            }
        }
        } else {
        for (int n = 0; n <= nsteps; ++n) {
            // block n has landed (block 1 may still fly at n = 0)
            if (n == 0 && nsteps > 1) wait_vm_n<LPS>();
            else wait_vm();
            __syncthreads();
            // copies of block n + 1 in two bursts: Q (+ a stats / delta row)
            // now, dO after the first sub-tile
            const bool cp = n >= 1 && n + 1 < nsteps;
            const int qn = q_top - (n + 1) * BQ;
            unsigned char* stn = smem + ((n + 1) % NSTAGE) * Cfg::STAGE;
            if (cp) {
                qd.issue(make_rsrc(Qb + (size_t)qn * D_qk, (long long)(S_q - qn) * D_qk * 2), stn, kw);
                if (kw == 0) dma4(make_rsrc(st2b + qn, (long long)(S_q - qn) * 4), stn + Cfg::QB + Cfg::OB, lane * 4);
                if (kw == 1)
                    dma4(make_rsrc(deltab + qn, (long long)(S_q - qn) * 4), stn + Cfg::QB + Cfg::OB + BQ * 4, lane * 4);
            }
            // block n has landed: its delta row becomes delta' (read by this
            // role from the next step on; the P role never reads it)
            if (DROP && kw == 1 && n < nsteps && !drop_all) {
                float* dl = reinterpret_cast<float*>(smem + (n % NSTAGE) * Cfg::STAGE + Cfg::QB + Cfg::OB) + BQ;
                dl[lane] = dl[lane] / ksc;
            }
            if (n == 0) continue;
            const int m = n - 1;
            const int q0 = q_top - m * BQ;
            const uint32_t qbase = (uint32_t)((m % NSTAGE) * Cfg::STAGE);
            half8 a0, a1, c0, c1;
            const bool l0 = sub_live(q0), l1 = sub_live(q0 + 32);
            if (l0) sub(qbase, m, 0, a0, a1);
            if (cp) od.issue(make_rsrc(dOb + (size_t)qn * D_v, (long long)(S_q - qn) * D_v * 2), stn + Cfg::QB, kw);
            if (l1) sub(qbase, m, 1, c0, c1);
            if constexpr (DS) {
                if (l0) store_ds(m, 0, a0, a1);
                if (l1) store_ds(m, 1, c0, c1);
            }
        }
        }
        if (key_ok) {
            half_t* dKb = static_cast<half_t*>(p.dk) + ((size_t)b * S_kv + my_k) * D_qk;
            const float fk = DROP && !drop_all ? p.c.scale * ksc : p.c.scale;
            if (D_qk == DQK) store_rows_f16<DQK>(dKb, dkacc, fk, hh);
            else store_rows_f16_n<DQK>(dKb, dkacc, fk, hh, D_qk);
        }
    }
}

}  // namespace

hipError_t launch_bwd_dkdv_f16_split(const BwdParams& p, hipStream_t stream) {
    const int B = p.s.B, S_kv = p.s.S_kv;
    if (B == 0 || S_kv == 0) return hipSuccess;
    return with_dim(p.s.D_qk, [&](auto dqk) {
        return with_dim(p.s.D_v, [&](auto dv) {
            return with_bool(p.c.causal != 0, [&](auto c) {
                return with_bool(p.c.use_dropout != 0, [&](auto d) {
                    constexpr int DQK = decltype(dqk)::value, DV = decltype(dv)::value;
                    constexpr bool CA = decltype(c)::value, DR = decltype(d)::value;
                    if constexpr (DQK == 128 || DV == 128) {
                        using CS = DkvSplitCfg<DQK, DV>;
                        static_assert(CS::BKV == DsLayout::KT && CS::BQ == DsLayout::QBK, "dS chunk geometry");
                        const long long n = (long long)((S_kv + CS::BKV - 1) / CS::BKV) * B;
                        const int win = row_window((size_t)p.s.S_q * (DQK + DV) * 2);
                        if (p.ds)
                            return launch_kernel<sdpa_bwd_dkdv_f16_split_kernel<DQK, DV, CA, DR, true>>(
                                (unsigned)n, CS::NT, CS::LDS_BYTES, stream, p, win);
                        return launch_kernel<sdpa_bwd_dkdv_f16_split_kernel<DQK, DV, CA, DR, false>>(
                            (unsigned)n, CS::NT, CS::LDS_BYTES, stream, p, win);
                    } else {
                        return hipErrorInvalidValue;  // the one-wave kernel serves D <= 64
                    }
                });
            });
        });
    });
}

}  // namespace sdpa
