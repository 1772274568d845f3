// sdpa_f16_fwd.hip -- fp16 Sdpa forward for gfx950 with its K/V tiles
// streamed from HBM straight into LDS (copy machinery in sdpa_dma.h).
//
// The production forward for the fp16 op whenever every feature width is a
// multiple of 8 and every tensor is 16-byte aligned; other fp16 shapes use the
// register-staged kernel of sdpa_fwd.hip.  Element semantics are those of the
// reference (sdpa/sdpa_fwd.cu.cc:93-173), restated in sdpa_fwd.hip.
//
// Per wave of 32 queries (lane = query), v_mfma_f32_32x32x16_f16 with fp32
// accumulation (lane layouts in sdpa_device.h):
//   S^T = K Q^T, online softmax over keys in the log2 domain,
//   O^T += V^T P~^T with P~ taken from the S accumulator straight into the B
//   operand of the PV MFMA.
// Four waves (128 queries) per workgroup, two workgroups per CU (three at
// D <= 64 without dropout), stream
// blocks of 64 keys through an LDS ring (three deep when it fits, else two),
// one barrier per block: each block's copy is issued one or two steps before
// it is read.
// Workgroup ids are remapped XCD-major (xcd_map); under causal masking the
// heaviest query tiles of a batch row run first.
//
// Instruction economy: the issue rate, not the MFMA pipe, bounds this kernel
// (the softmax and dropout cost ~8 VALU operations per score against 0.5
// MFMA clocks), so a step carries little address arithmetic: every LDS read
// is one v_xad of a lane term and the stage base, with the row offsets as
// instruction immediates, and a tile copy needs scalar descriptors only.
//
// Built without IEEE mode (-mno-amdgpu-ieee -fno-honor-nans): the row maxima
// then take one v_max3 per two scores instead of first canonicalising every
// operand.  Inputs are finite; NaN inputs propagate differently than in
// IEEE mode.
#include <type_traits>

#include "sdpa_dma.h"
#include "sdpa_launch.h"
#include "sdpa_params.h"

namespace sdpa {
namespace {

// Lazy-rescale threshold of the running maximum (log2 units).
constexpr float kTauF = 8.0f;

template <int DQK, int DV>
struct FwdDmaCfg {
    // NW waves of 32 queries each; K/V blocks of BN keys in an NSTAGE-deep
    // LDS ring (the copy of block n + NSTAGE - 1 is issued at step n).  Two
    // or three workgroups share a CU, so the waves on a SIMD belong to different
    // workgroups and never wait at each other's barriers (a workgroup of
    // eight waves, two per SIMD, measured slower: each step the older wave
    // finishes first and the other then runs alone).
    static constexpr int NW = 4, NT = 64 * NW, BM = 32 * NW, BN = 64;
    static constexpr int LK = DQK / 8, LV = DV / 8;
    static constexpr int KB = BN * DQK * 2, VB = BN * DV * 2, STAGE = KB + VB;
    static constexpr int NSTAGE = 2 * 3 * STAGE <= 160 * 1024 ? 3 : 2;
    static constexpr size_t LDS_BYTES = NSTAGE * (size_t)STAGE;
    static_assert(2 * LDS_BYTES <= 160 * 1024, "two workgroups per CU in gfx950 LDS");
    // waves per SIMD: three when three workgroups' LDS fits, D <= 64 and no
    // dropout (the register footprint then stays under 168 without spills)
    template <bool DROP>
    static constexpr int wpe() { return (!DROP && DQK <= 64 && DV <= 64 && 3 * LDS_BYTES <= 160 * 1024) ? 3 : 2; }
    // every read offset (tile + rows) fits the 16-bit DS immediate
    static_assert(KB + VB <= 65536, "LDS immediates");
};

template <int DQK, int DV, bool CAUSAL, bool DROP>
__global__ __launch_bounds__((FwdDmaCfg<DQK, DV>::NT))
__attribute__((amdgpu_waves_per_eu(FwdDmaCfg<DQK, DV>::template wpe<DROP>(), FwdDmaCfg<DQK, DV>::template wpe<DROP>())))
void sdpa_fwd_f16_dma_kernel(const FwdParams p, const int win) {
    using Cfg = FwdDmaCfg<DQK, DV>;
    constexpr int BM = Cfg::BM, BN = Cfg::BN, LK = Cfg::LK, LV = Cfg::LV, NW = Cfg::NW, NSTAGE = Cfg::NSTAGE;
    constexpr int NKS = DQK / 16, NDT = DV / 32;

    const int tid = threadIdx.x, lane = tid & 63, l32 = lane & 31, hh = lane >> 5;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int B = p.s.B, S_q = p.s.S_q, S_kv = p.s.S_kv, D_qk = p.s.D_qk, D_v = p.s.D_v;
    const int tiles = (S_q + BM - 1) / BM;
    int b, qt;
    xcd_map(blockIdx.x, B * tiles, tiles, CAUSAL, win, b, qt);
    const int q0 = qt * BM, qw0 = q0 + 32 * wave, my_q = qw0 + l32;

    const half_t* Qb = static_cast<const half_t*>(p.q) + (size_t)b * S_q * D_qk;
    // K/V rows of this batch row (scalar descriptors; see RowSrc)
    const RowSrc ksrc = row_src(p.k, (size_t)b * S_kv, S_kv, D_qk * 2);
    const RowSrc vsrc = row_src(p.v, (size_t)b * S_kv, S_kv, D_v * 2);

    // The running maximum is taken on raw scores q.k, which needs a
    // non-negative factor: for scale < 0 the queries are negated in
    // registers (exact) and |scale| used.  A zero factor is replaced by
    // 1e-30, which leaves every probability 1 to within 1e-26.
    const float sl2_raw = p.c.scale_log2;
    const bool neg = sl2_raw < 0.f;
    const float sl2 = (sl2_raw == 0.f) ? 1e-30f : fabsf(sl2_raw);

    half8 qreg[NKS];
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) {
        half8 v = __builtin_bit_cast(half8, load_row_chunk<half_t, true>(Qb, my_q, S_q, 16 * ks + 8 * hh, D_qk, D_qk));
        qreg[ks] = neg ? -v : v;
    }

    // ---- tile copies: one descriptor per tile, per-copy lane offsets fixed
    const int krow = D_qk * 2, vrow = D_v * 2;
    TileCopy<BN, LK, NW> kc;
    TileCopy<BN, LV, NW, true> vc;  // V is read only transposed
    kc.init(wave, lane, krow, D_qk / 8);
    vc.init(wave, lane, vrow, D_v / 8);
    const uint32_t lds0 = lds_base();
    const uint32_t m0w = lds0 + 1024u * (uint32_t)wave;
    const int kv_end = CAUSAL ? min(S_kv, q0 + BM) : S_kv;
    const int nsteps = (kv_end + BN - 1) / BN;
    // copy of key block `step` into its ring slot (step % NSTAGE)
    auto issue = [&](int step) {
        const int kv0 = step * BN;
        const uint32_t so = (uint32_t)((step % NSTAGE) * Cfg::STAGE);
        kc.issue(ksrc.shifted(kv0), m0w + so, wave);
        vc.issue(vsrc.shifted(kv0), m0w + so + (uint32_t)Cfg::KB, wave);
    };
    // copies this wave issues per block (its vmcnt waits count only those)
    const int cpb = TileCopy<BN, LK, NW>::count(wave) + TileCopy<BN, LV, NW, true>::count(wave);
#pragma unroll
    for (int i = 0; i < NSTAGE - 1; ++i)
        if (i < nsteps) issue(i);

    // ---- lane read addresses (the stage base and row offsets are added per
    // step / as instruction immediates).  The swizzle only permutes 16-byte
    // chunks inside a row and stage bases are multiples of 4 KB, so a read
    // address is (lane term ^ chunk term) + stage base: one v_xad each.
    SwzLane<LK> swK;
    swK.init(lane);
    const uint32_t rkl = lds0 + swK.row;                              // K rows (^ 32 ks)
    const uint32_t tvl = lds0 + Cfg::KB + tr_lane_off<LV>(lane);      // V^T (^ 64 dt)

    floatx16 oacc[NDT];
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) oacc[dt] = floatx16{};
    float m_run = kMaxSentinel, l_run = 0.f;

    // Dropout hash of (my_q, key 4 hh); element (key kv0 + c) adds (kv0 + c) A.
    // st_blk walks the key blocks: + BN A per step.
    uint64_t st_blk = DROP ? lcg_state(p.c.seed_offset, (uint64_t)b * S_q + my_q, (uint64_t)S_kv, 4 * hh) : 0;
    const uint32_t thr = p.c.drop_threshold;

    // Softmax of one 32-key sub-tile t (scores s, raw q.k; masked keys set to
    // -inf by the caller): per-lane lazy maximum m_use (moves only when the
    // block maximum exceeds the running one by more than 2^kTauF), alpha =
    // exp2(m_run - m_use), P = exp2(s sl2 - m_use), the undropped sum and the
    // dropped, fp16-packed B operands of the PV product; also the row maximum
    // mxo (log2 units) and the dropped P~ in fp32 (pf, for the hi/lo split).
    auto softmax_sub = [&](const floatx16& sc, int t, uint64_t st_blk, float& m_use, float& alpha, float& lsum,
                           float& mxo, half8& pb0, half8& pb1, float (&pf)[16]) {
        // a chain of v_max3 (one per two scores): the opaque steps keep the
        // compiler from re-associating it into a tree of v_max and v_max3,
        // which costs ~1.4 instructions per two scores
        float mx = fmaxf(fmaxf(sc[0], sc[1]), sc[2]);
#pragma unroll
        for (int r = 3; r < 15; r += 2) {
            asm("" : "+v"(mx));
            mx = fmaxf(mx, fmaxf(sc[r], sc[r + 1]));
        }
        mx = fmaxf(mx, sc[15]);
        mx = xhalf_max(mx) * sl2;
        mxo = mx;
        m_use = (mx > m_run + kTauF) ? fmaxf(m_run, mx) : m_run;
        alpha = fast_exp2(m_run - m_use);
        const float nm = -m_use;
        uint32_t w[8];
        float lq[4];
        // Hash states walk the lane's keys 32 t + 8 g + e as a chain of adds
        // (opaque to the compiler, which would otherwise fold them into 32
        // distinct 64-bit constants and run out of scalar registers).
        uint64_t sg = DROP ? st_blk + (uint64_t)(32 * t) * kLcgMul : 0;
#pragma unroll
        for (int r = 0; r < 16; r += 4) {
            float pq[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) pq[e] = fast_exp2(__builtin_fmaf(sc[r + e], sl2, nm));
            lq[r >> 2] = (pq[0] + pq[1]) + (pq[2] + pq[3]);
            if constexpr (DROP) {
                uint64_t se = sg;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    pq[e] = lcg_keep(se, thr) ? pq[e] : 0.f;
                    if (e < 3) {
                        se += kLcgMul;
                        asm volatile("" : "+v"(se));
                    }
                }
                sg += 8 * kLcgMul;
                asm volatile("" : "+v"(sg));
            }
            w[r >> 1] = pack_h2(pq[0], pq[1]);
            w[(r >> 1) + 1] = pack_h2(pq[2], pq[3]);
#pragma unroll
            for (int e = 0; e < 4; ++e) pf[r + e] = pq[e];
        }
        lsum = (lq[0] + lq[1]) + (lq[2] + lq[3]);
        pb0 = half8_of(w[0], w[1], w[2], w[3]);
        pb1 = half8_of(w[4], w[5], w[6], w[7]);
    };
    // The lo part of a split sub-tile: O^T += V^T (P~ - fp16(P~))^T.
    auto lo_pv = [&](const half8 (&av)[2][NDT], const half8& pb0, const half8& pb1, const float (&pf)[16]) {
        uint32_t wl[8];
#pragma unroll
        for (int i = 0; i < 8; i += 2) {
            wl[i >> 1] = pack_h2(pf[i] - (float)pb0[i], pf[i + 1] - (float)pb0[i + 1]);
            wl[4 + (i >> 1)] = pack_h2(pf[8 + i] - (float)pb1[i], pf[9 + i] - (float)pb1[i + 1]);
        }
        const half8 l0 = half8_of(wl[0], wl[1], wl[2], wl[3]), l1 = half8_of(wl[4], wl[5], wl[6], wl[7]);
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) {
            oacc[dt] = mfma_f16(av[0][dt], l0, oacc[dt]);
            oacc[dt] = mfma_f16(av[1][dt], l1, oacc[dt]);
        }
    };
    // Mask of sub-tile t: keys past S_kv and, causal, keys after the query.
    auto mask_sub = [&](floatx16& sc, int kv0, int t) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int key = kv0 + 32 * t + 8 * (r >> 2) + 4 * hh + (r & 3);
            if (key >= S_kv || (CAUSAL && key > my_q)) sc[r] = -INFINITY;
        }
    };
    // After a sub-tile's PV operands are formed: rescale the output (rare,
    // wave-uniform branch) and fold the sub-tile into the running sum.
    auto commit_sub = [&](float m_use, float alpha, float lsum) {
        if (wave_any(alpha != 1.f)) {
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
                for (int r = 0; r < 16; ++r) oacc[dt][r] *= alpha;
        }
        l_run = __builtin_fmaf(l_run, alpha, lsum);
        m_run = m_use;
    };

    // One step = 64 keys (stage at byte offset so) as two 32-key sub-tiles, written in
    // software-pipeline order so that each MFMA group has independent work
    // next to it (a wave issues in order; the compiler interleaves within
    // these spans):
    //   R1  S(0) = K0 Q^T           with LDS reads of K1
    //   R2  S(1) = K1 Q^T           with softmax(0), LDS reads of V0^T
    //   R3  O^T += V0^T P0~^T       with softmax(1), LDS reads of V1^T
    //   R4  O^T += V1^T P1~^T
    // The rescale of O by sub-tile 1's new maximum commutes with the pending
    // PV(0) accumulation, so it is applied after R3.
    // mid(k) marks the end of region k (the copy points of the step).
    //
    // A sub-tile whose largest score passes the row's split threshold thr
    // (the running log2-sum-exp before this step + kSplitLog2; -inf before
    // any key) also adds its lo part (lo_pv, a rare wave-uniform branch).
    auto fwd_step = [&]<bool PART>(int kv0, uint32_t so, auto&& mid) {
        const bool part0 = PART && (kv0 + 32 > S_kv || (CAUSAL && kv0 + 31 > qw0));
        const bool part1 = PART && (kv0 + 64 > S_kv || (CAUSAL && kv0 + 63 > qw0));
        const float thr = m_run + fast_log2(xhalf_sum(l_run)) + kSplitLog2;
        // Read addresses of this step, formed here (opaque lane terms keep the
        // compiler from hoisting twelve of them into registers for the loop).
        uint32_t kl = rkl, vl = tvl;
        asm volatile("" : "+v"(kl), "+v"(vl));
        uint32_t rk[NKS], tv[NDT];
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks) rk[ks] = (kl ^ (uint32_t)(32 * ks)) + so;
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) tv[dt] = (vl ^ (uint32_t)(64 * dt)) + so;
        half8 ak0[NKS], ak1[NKS];
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks) ak0[ks] = ld_b128(rk[ks]);
        // R1
        floatx16 s0 = floatx16{}, s1 = floatx16{};
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks) {
            s0 = mfma_f16(ak0[ks], qreg[ks], s0);
            ak1[ks] = ld_b128(rk[ks] + 16 * LK * 32);
        }
        mid(1);
        // R2
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks) s1 = mfma_f16(ak1[ks], qreg[ks], s1);
        half8 av0[2][NDT], av1[2][NDT];
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt)
                av0[j][dt] = ld_tr8(tv[dt] + 16 * LV * 16 * j, tv[dt] + 16 * LV * (16 * j + 8));
        if (part0) mask_sub(s0, kv0, 0);
        float mu0, al0, ls0, mx0, pf0[16];
        half8 p00, p01;
        softmax_sub(s0, 0, st_blk, mu0, al0, ls0, mx0, p00, p01, pf0);
        commit_sub(mu0, al0, ls0);
        mid(2);
        // R3
        if (wave_any(mx0 > thr)) lo_pv(av0, p00, p01, pf0);
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) {
            oacc[dt] = mfma_f16(av0[0][dt], p00, oacc[dt]);
            oacc[dt] = mfma_f16(av0[1][dt], p01, oacc[dt]);
        }
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt)
                av1[j][dt] = ld_tr8(tv[dt] + 16 * LV * (32 + 16 * j), tv[dt] + 16 * LV * (40 + 16 * j));
        if (part1) mask_sub(s1, kv0, 1);
        float mu1, al1, ls1, mx1, pf1[16];
        half8 p10, p11;
        softmax_sub(s1, 1, st_blk, mu1, al1, ls1, mx1, p10, p11, pf1);
        commit_sub(mu1, al1, ls1);
        mid(3);
        // R4
        if (wave_any(mx1 > thr)) lo_pv(av1, p10, p11, pf1);
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) {
            oacc[dt] = mfma_f16(av1[0][dt], p10, oacc[dt]);
            oacc[dt] = mfma_f16(av1[1][dt], p11, oacc[dt]);
        }
    };

    // Step `step`: wait for its block (the copies of the NSTAGE - 2 later
    // blocks may still fly; all of them at the tail), synchronise, multiply,
    // and copy block step + NSTAGE - 1 into the slot of block step - 1 (every
    // wave has finished reading it).  Waves 0 and 1 issue their copies right
    // after the barrier, waves 2 and 3 after R1.  Issued by all four there,
    // they queue behind each other in the CU's address unit and stall all
    // four waves at once; spread over four points (the barrier, after R1, R2
    // and R3), the last wave's copies had only R4 to land before the next
    // step waits for them.  Only the copy point after R1 stays in the step's
    // code: a copy branch at the end of R2 or R3 also splits the compiler's
    // scheduling regions there (with them compiled in but never taken, c4's
    // forward took 0.717 against 0.695 ms; with four points, 0.711 ms).
    const bool live = qw0 < S_q;
    auto do_step = [&]<bool PART>(int step) {
        const uint32_t so = (uint32_t)((step % NSTAGE) * Cfg::STAGE);
        if (step + NSTAGE - 2 < nsteps) wait_vm_upto((NSTAGE - 2) * cpb);
        else wait_vm();
        __syncthreads();
        const bool cp = step + NSTAGE - 1 < nsteps;
        static_assert(NW == 4, "copy points of four waves");
        const bool late = wave >= 2;  // issues after R1
        if (cp && !late) issue(step + NSTAGE - 1);
        const int kv0 = step * BN;
        auto mid = [&](int k) {
            if (k == 1 && cp && late) issue(step + NSTAGE - 1);
        };
        if (!PART || (live && !(CAUSAL && kv0 > qw0 + 31))) {  // else: no visible key in this step
            fwd_step.template operator()<PART>(kv0, so, mid);
        }
        else if (cp && late)
            issue(step + NSTAGE - 1);
        if constexpr (DROP) st_blk += (uint64_t)BN * kLcgMul;
    };
    // Steps whose 64 keys are all visible to all 32 queries of this wave run
    // the unmasked variant; the causal diagonal and the key tail come last.
    const int full_lim = CAUSAL ? min(qw0 - (BN - 1), S_kv - BN) : S_kv - BN;
    const int n_full = qw0 >= S_q ? 0 : min(nsteps, full_lim < 0 ? 0 : full_lim / BN + 1);
    int step = 0;
    for (; step < n_full; ++step) do_step.template operator()<false>(step);
    for (; step < nsteps; ++step) do_step.template operator()<true>(step);

    // ---- epilogue: stats = m + log(l + 1e-6), O = acc / l (0 if l <= 1e-6) ----
    const float l_tot = xhalf_sum(l_run);
    if (my_q < S_q) {
        const float m_nat = (l_tot > 0.f) ? m_run * kLn2 : kNegInf;
        if (hh == 0) p.stats[(size_t)b * S_q + my_q] = m_nat + logf(l_tot + kEps);
        const float inv = (l_tot > kEps) ? p.c.keep_scale / l_tot : 0.f;
        half_t* Ob = static_cast<half_t*>(p.o) + ((size_t)b * S_q + my_q) * D_v;
        if (D_v == DV) store_rows_f16<DV>(Ob, oacc, inv, hh);
        else store_rows_f16_n<DV>(Ob, oacc, inv, hh, D_v);
    }
}

}  // namespace

hipError_t launch_fwd_f16_dma(const FwdParams& p, hipStream_t stream) {
    const int B = p.s.B, S_q = p.s.S_q;
    if (B == 0 || S_q == 0) return hipSuccess;
    return with_dim(p.s.D_qk, [&](auto dqk) {
        return with_dim(p.s.D_v, [&](auto dv) {
            return with_bool(p.c.causal != 0, [&](auto c) {
                return with_bool(p.c.use_dropout != 0, [&](auto d) {
                    constexpr int DQK = decltype(dqk)::value, DV = decltype(dv)::value;
                    using Cfg = FwdDmaCfg<DQK, DV>;
                    const long long n = (long long)((S_q + Cfg::BM - 1) / Cfg::BM) * B;
                    return launch_kernel<sdpa_fwd_f16_dma_kernel<DQK, DV, decltype(c)::value, decltype(d)::value>>(
                        (unsigned)n, Cfg::NT, Cfg::LDS_BYTES, stream, p,
                        row_window((size_t)p.s.S_kv * (DQK + DV) * 2));
                });
            });
        });
    });
}

}  // namespace sdpa
