// sdpa_fwd.hip -- forward kernels of the Sdpa op for gfx950.
//
// Replaces FlashAttnFwdKernel + FlashAttnFunctor<GPUDevice,T>
// (sdpa/sdpa_fwd.cu.cc:11-240) with a workgroup-tiled online softmax on MFMA.
//
// Work decomposition (both dtypes): a workgroup of 4 waves owns BM = 128
// consecutive queries of one batch row; each wave owns 32 of them and keeps
// its Q rows in registers for the whole kernel.  K/V blocks of BN keys are
// staged through LDS (double buffered: the global loads of block n+1 are in
// flight while block n is multiplied).  Per block each wave computes
//   S^T = K Q^T              (keys x queries, C layout: one query per lane)
//   online softmax over keys (in-lane max/sum + one permlane32 swap)
//   O^T += V^T P~^T          (P~ taken straight from the S^T accumulator)
// so row statistics never leave the lane and P never touches LDS.
//
// Semantics kept from the reference (sdpa/sdpa_fwd.cu.cc):
//   - causal mask top-left aligned, key j visible to query i iff j <= i (:93-96)
//   - the denominator l sums undropped probabilities (:134-135)
//   - stats = m + log(l + 1e-6) (:160), o = acc / l if l > 1e-6 else 0 (:163)
//   - dropout element (b,i,j) keyed on the reference's LCG hash (:136-146)
// The exp is evaluated as exp2 of log2-scaled scores; the running maximum is
// updated lazily (only when it grows by more than kTau in log2 units), which
// changes rounding only: o and stats are invariant to the reference point.
#include <mutex>
#include <type_traits>

#include "sdpa_device.h"
#include "sdpa_launch.h"
#include "sdpa_params.h"
#include "sdpa_tile.h"

namespace sdpa {

constexpr float kTau = 8.0f;  // lazy-rescale threshold (log2 units): p <= 2^8

// Workgroup -> (batch, query tile).  Causal tiles are issued heaviest first
// (the last query tiles see the most keys); consecutive workgroup ids walk
// the batch, so with B a multiple of 8 every tile of batch b is dispatched to
// the same XCD (ids are dealt round-robin over the 8 XCDs) and shares that
// XCD's L2 copy of K and V.
__device__ __forceinline__ void map_q_tile(int bid, int B, int tiles, bool causal, int& b, int& t) {
    b = bid % B;
    const int level = bid / B;
    t = causal ? (tiles - 1 - level) : level;
}

// ---------------------------------------------------------------------------
// fp16: v_mfma_f32_32x32x16_f16, fp32 accumulation.
// ---------------------------------------------------------------------------
template <int DQK, int DV>
struct FwdF16Cfg {
    static constexpr int NT = 256, BM = 128, BN = 64;
    // K and V tiles are unpadded and chunk-swizzled (swz_off): K is read by
    // rows (b128), V by transpose reads; both are bank-conflict-free.
    static constexpr int KT = BN * DQK, VT = BN * DV, STAGE = KT + VT;
    static constexpr size_t LDS_BYTES = 2 * (size_t)STAGE * sizeof(half_t);
};

// Two waves per SIMD throughout: with the split pass in the block loop,
// <128,128> with dropout keeps 32 (aligned rows) and 88 (generic row loads)
// bytes per lane in scratch, every other instantiation none; one wave per
// SIMD, spill-free, measured 5-6.5% slower at D = 124 and 60 / 124.
template <int DQK, int DV, bool VEC, bool DROP>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2)))
void sdpa_fwd_f16_kernel(const FwdParams p) {
    using Cfg = FwdF16Cfg<DQK, DV>;
    constexpr int BM = Cfg::BM, BN = Cfg::BN, LK = DQK / 8, LV = DV / 8;
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    half_t* lds = reinterpret_cast<half_t*>(smem);

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int l32 = lane & 31, hh = lane >> 5;
    const int B = p.s.B, S_q = p.s.S_q, S_kv = p.s.S_kv, D_qk = p.s.D_qk, D_v = p.s.D_v;
    const bool causal = p.c.causal != 0;
    const int tiles = (S_q + BM - 1) / BM;
    int b, qt;
    map_q_tile(blockIdx.x, B, tiles, causal, b, qt);
    const int q0 = qt * BM, qw0 = q0 + wave * 32, my_q = qw0 + l32;

    const half_t* Qb = static_cast<const half_t*>(p.q) + (size_t)b * S_q * D_qk;
    const half_t* Kb = static_cast<const half_t*>(p.k) + (size_t)b * S_kv * D_qk;
    const half_t* Vb = static_cast<const half_t*>(p.v) + (size_t)b * S_kv * D_v;

    // Q^T as the B operand: lane holds query my_q, features 16ks + 8hh .. +7.
    half8 qreg[DQK / 16];
#pragma unroll
    for (int ks = 0; ks < DQK / 16; ++ks) {
        const uint4 c = load_row_chunk<half_t, VEC>(Qb, my_q, S_q, 16 * ks + 8 * hh, D_qk, D_qk);
        qreg[ks] = __builtin_bit_cast(half8, c);
    }
    prologue_loads_landed();

    const int kv_end = causal ? min(S_kv, q0 + BM) : S_kv;
    const int nblk = (kv_end + BN - 1) / BN;
    const bool wave_live = qw0 < S_q;
    const int wave_last_q = min(qw0 + 31, S_q - 1);

    floatx16 oacc[DV / 32];
#pragma unroll
    for (int dt = 0; dt < DV / 32; ++dt) oacc[dt] = floatx16{};
    float m_run = kMaxSentinel, l_run = 0.f;
    const float sl2 = p.c.scale_log2;

    // Dropout hash state of (my_q, key 4*hh); element offsets are constants.
    const uint64_t st_base =
        DROP ? lcg_state(p.c.seed_offset, (uint64_t)b * S_q + my_q, (uint64_t)S_kv, 4 * hh) : 0;
    const uint32_t thr = p.c.drop_threshold;

    // Transpose-read coordinates (see lds_read_tr): 16-lane group g reads
    // key rows 4*(g/2) + i/4 and feature columns 16*(g%2) + 4*(i%4).
    const int g16 = lane >> 4, i16 = lane & 15;
    const int tr_row = 4 * (g16 >> 1) + (i16 >> 2);
    const int tr_col = 16 * (g16 & 1) + 4 * (i16 & 3);

    TileStage<half_t, BN, DQK, Cfg::NT, VEC> kst;
    TileStage<half_t, BN, DV, Cfg::NT, VEC> vst;
    if (nblk > 0) {
        kst.load(Kb, 0, S_kv, D_qk, D_qk, tid);
        vst.load(Vb, 0, S_kv, D_v, D_v, tid);
        kst.store_swz(lds, tid);
        vst.store_swz(lds + Cfg::KT, tid);
    }
    __syncthreads();

    // S^T = K Q^T of one key block, log2-scaled, masked keys -inf.
    auto scores = [&](floatx16 (&sacc)[BN / 32], const half_t* Ks, int kv0) {
#pragma unroll
        for (int t = 0; t < BN / 32; ++t) sacc[t] = floatx16{};
#pragma unroll
        for (int ks = 0; ks < DQK / 16; ++ks) {
#pragma unroll
            for (int t = 0; t < BN / 32; ++t) {
                const half8 a = *reinterpret_cast<const half8*>(Ks + swz_off<LK>(32 * t + l32, 16 * ks + 8 * hh));
                sacc[t] = mfma_f16(a, qreg[ks], sacc[t]);
            }
        }
        const bool need_mask = (kv0 + BN > S_kv) || (causal && kv0 + BN - 1 > qw0);
#pragma unroll
        for (int t = 0; t < BN / 32; ++t) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                float x = sacc[t][r] * sl2;
                if (need_mask) {
                    const int key = kv0 + 32 * t + 8 * (r >> 2) + 4 * hh + (r & 3);
                    if (key >= S_kv || (causal && key > my_q)) x = -INFINITY;
                }
                sacc[t][r] = x;
            }
        }
    };
    // P~ = exp2(s - m_run) with dropout, as fp16 B operands of the PV product:
    // LO = false the values (pb; the undropped sum goes into l_run), LO = true
    // their remainders P~ - fp16(P~) (the lo part of the hi/lo split).
    auto probs = [&]<bool LO>(const floatx16 (&sacc)[BN / 32], int kv0, half8 (&pb)[BN / 16]) {
        const uint64_t st_blk = DROP ? st_base + (uint64_t)kv0 * kLcgMul : 0;
        float lsum = 0.f;
#pragma unroll
        for (int t = 0; t < BN / 32; ++t) {
#pragma unroll
            for (int r = 0; r < 16; r += 2) {
                float p0 = fast_exp2(sacc[t][r] - m_run);
                float p1 = fast_exp2(sacc[t][r + 1] - m_run);
                lsum += p0;
                lsum += p1;
                if constexpr (DROP) {
                    const uint64_t o0 = (uint64_t)(32 * t + 8 * (r >> 2) + (r & 3)) * kLcgMul;
                    const uint64_t o1 = (uint64_t)(32 * t + 8 * ((r + 1) >> 2) + ((r + 1) & 3)) * kLcgMul;
                    p0 = lcg_keep(st_blk + o0, thr) ? p0 : 0.f;
                    p1 = lcg_keep(st_blk + o1, thr) ? p1 : 0.f;
                }
                half2v hp = cvt_pk(p0, p1);
                if constexpr (LO) hp = cvt_pk(p0 - (float)hp[0], p1 - (float)hp[1]);
                const int s = 2 * t + (r >> 3), i = r & 7;
                pb[s][i] = hp[0];
                pb[s][i + 1] = hp[1];
            }
        }
        if constexpr (!LO) l_run += lsum;
    };
    // O^T += V^T P~^T
    auto pv = [&](const half_t* Vs, const half8 (&pb)[BN / 16]) {
#pragma unroll
        for (int s = 0; s < BN / 16; ++s) {
#pragma unroll
            for (int dt = 0; dt < DV / 32; ++dt) {
                const half4 a0 = lds_read_tr(Vs + swz_off<LV>(16 * s + tr_row, 32 * dt + tr_col));
                const half4 a1 = lds_read_tr(Vs + swz_off<LV>(16 * s + 8 + tr_row, 32 * dt + tr_col));
                const half8 a = __builtin_shufflevector(a0, a1, 0, 1, 2, 3, 4, 5, 6, 7);
                oacc[dt] = mfma_f16(a, pb[s], oacc[dt]);
            }
        }
    };

    // One key block.  The hi/lo split of P~ (sdpa_device.h, kSplitLog2) is
    // decided per block: when some row's block maximum passes its running
    // log2-sum-exp (before the block) + kSplitLog2, the block's lo part is
    // added after the next block's tiles have left their staging registers
    // for LDS: S and P~ are formed again from the block's LDS tiles (same
    // instructions on the same operands: the same values), so that nothing
    // of the first pass stays live across it.
    auto block = [&](int blk) {
        const int kv0 = blk * BN;
        const half_t* Ks = lds + (blk & 1) * Cfg::STAGE;
        const half_t* Vs = Ks + Cfg::KT;
        const bool has_next = blk + 1 < nblk;
        if (has_next) {
            kst.load(Kb, kv0 + BN, S_kv - kv0 - BN, D_qk, D_qk, tid);
            vst.load(Vb, kv0 + BN, S_kv - kv0 - BN, D_v, D_v, tid);
        }

        bool split = false;
        if (wave_live && (!causal || kv0 <= wave_last_q)) {
            const float split_thr = m_run + fast_log2(xhalf_sum(l_run)) + kSplitLog2;
            floatx16 sacc[BN / 32];
            scores(sacc, Ks, kv0);
            float mx = -INFINITY;
#pragma unroll
            for (int t = 0; t < BN / 32; ++t)
#pragma unroll
                for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sacc[t][r]);
            mx = xhalf_max(mx);
            split = wave_any(mx > split_thr);
            const float m_new = fmaxf(m_run, mx);
            if (wave_any(m_new > m_run + kTau)) {
                const float alpha = fast_exp2(m_run - m_new);
                l_run *= alpha;
#pragma unroll
                for (int dt = 0; dt < DV / 32; ++dt)
#pragma unroll
                    for (int r = 0; r < 16; ++r) oacc[dt][r] *= alpha;
                m_run = m_new;
            }
            half8 pb[BN / 16];
            probs.template operator()<false>(sacc, kv0, pb);
            pv(Vs, pb);
        }

        if (has_next) {
            half_t* Kn = lds + ((blk + 1) & 1) * Cfg::STAGE;
            kst.store_swz(Kn, tid);
            vst.store_swz(Kn + Cfg::KT, tid);
        }
        if (split) {
            // opaque copies of the tile offset and key index: nothing here
            // is merged with the first pass
            int z = 0, kz = kv0;
            asm volatile("" : "+s"(z), "+s"(kz));
            floatx16 sacc[BN / 32];
            scores(sacc, Ks + z, kz);
            half8 pl[BN / 16];
            probs.template operator()<true>(sacc, kz, pl);
            pv(Vs + z, pl);
        }
        __syncthreads();
    };
    for (int blk = 0; blk < nblk; ++blk) block(blk);

    // ---- epilogue: stats and O = acc / l ----------------------------------
    const float l_tot = xhalf_sum(l_run);
    if (my_q < S_q) {
        const float m_nat = (l_tot > 0.f) ? m_run * kLn2 : kNegInf;
        if (hh == 0) p.stats[(size_t)b * S_q + my_q] = m_nat + logf(l_tot + kEps);
        const float inv = (l_tot > kEps) ? p.c.keep_scale / l_tot : 0.f;
        half_t* Ob = static_cast<half_t*>(p.o) + ((size_t)b * S_q + my_q) * D_v;
#pragma unroll
        for (int dt = 0; dt < DV / 32; ++dt) {
#pragma unroll
            for (int g4 = 0; g4 < 4; ++g4) {
                const int d0 = 32 * dt + 8 * g4 + 4 * hh;
                half4 hv;
#pragma unroll
                for (int e = 0; e < 4; ++e) hv[e] = (half_t)(oacc[dt][4 * g4 + e] * inv);
                if constexpr (VEC) {
                    if (d0 < D_v) *reinterpret_cast<half4*>(Ob + d0) = hv;
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (d0 + e < D_v) Ob[d0 + e] = hv[e];
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------
// fp32: v_mfma_f32_32x32x2_f32.  The reduction over features is split between
// the two half-waves: lane-half h covers features [h*DQK/2, (h+1)*DQK/2), so
// both K (LDS) and Q (registers) are read as contiguous float4 runs.
// ---------------------------------------------------------------------------
template <int DQK, int DV>
struct FwdF32Cfg {
    static constexpr int NT = 256, BM = 128, BN = 32;
    static constexpr int KS = DQK + 4;  // float4 reads by 16 rows hit 64 distinct banks
    static constexpr int VS = DV + 8;   // the two half-waves read rows 4 apart: disjoint banks
    static constexpr int KT = BN * KS, VT = BN * VS, STAGE = KT + VT;
    static constexpr size_t LDS_BYTES = 2 * (size_t)STAGE * sizeof(float);
};

template <int DQK, int DV, bool VEC, bool DROP>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2)))
void sdpa_fwd_f32_kernel(const FwdParams p) {
    using Cfg = FwdF32Cfg<DQK, DV>;
    constexpr int BM = Cfg::BM, BN = Cfg::BN, KS = Cfg::KS, VS = Cfg::VS;
    constexpr int HQ = DQK / 2;  // features per half-wave
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    float* lds = reinterpret_cast<float*>(smem);

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int l32 = lane & 31, hh = lane >> 5;
    const int B = p.s.B, S_q = p.s.S_q, S_kv = p.s.S_kv, D_qk = p.s.D_qk, D_v = p.s.D_v;
    const bool causal = p.c.causal != 0;
    const int tiles = (S_q + BM - 1) / BM;
    int b, qt;
    map_q_tile(blockIdx.x, B, tiles, causal, b, qt);
    const int q0 = qt * BM, qw0 = q0 + wave * 32, my_q = qw0 + l32;

    const float* Qb = static_cast<const float*>(p.q) + (size_t)b * S_q * D_qk;
    const float* Kb = static_cast<const float*>(p.k) + (size_t)b * S_kv * D_qk;
    const float* Vb = static_cast<const float*>(p.v) + (size_t)b * S_kv * D_v;

    float qf[HQ];
#pragma unroll
    for (int u = 0; u < HQ / 4; ++u) {
        const uint4 c = load_row_chunk<float, VEC>(Qb, my_q, S_q, HQ * hh + 4 * u, D_qk, D_qk);
        const floatx4 f = __builtin_bit_cast(floatx4, c);
#pragma unroll
        for (int e = 0; e < 4; ++e) qf[4 * u + e] = f[e];
    }
    prologue_loads_landed();

    const int kv_end = causal ? min(S_kv, q0 + BM) : S_kv;
    const int nblk = (kv_end + BN - 1) / BN;
    const bool wave_live = qw0 < S_q;
    const int wave_last_q = min(qw0 + 31, S_q - 1);

    floatx16 oacc[DV / 32];
#pragma unroll
    for (int dt = 0; dt < DV / 32; ++dt) oacc[dt] = floatx16{};
    float m_run = kMaxSentinel, l_run = 0.f;
    const float sl2 = p.c.scale_log2;
    const uint64_t st_base =
        DROP ? lcg_state(p.c.seed_offset, (uint64_t)b * S_q + my_q, (uint64_t)S_kv, 4 * hh) : 0;
    const uint32_t thr = p.c.drop_threshold;

    TileStage<float, BN, DQK, Cfg::NT, VEC> kst;
    TileStage<float, BN, DV, Cfg::NT, VEC> vst;
    if (nblk > 0) {
        kst.load(Kb, 0, S_kv, D_qk, D_qk, tid);
        vst.load(Vb, 0, S_kv, D_v, D_v, tid);
        kst.template store<KS>(lds, tid);
        vst.template store<VS>(lds + Cfg::KT, tid);
    }
    __syncthreads();

    for (int blk = 0; blk < nblk; ++blk) {
        const int kv0 = blk * BN;
        const float* Ks = lds + (blk & 1) * Cfg::STAGE;
        const float* Vs = Ks + Cfg::KT;
        const bool has_next = blk + 1 < nblk;
        if (has_next) {
            kst.load(Kb, kv0 + BN, S_kv - kv0 - BN, D_qk, D_qk, tid);
            vst.load(Vb, kv0 + BN, S_kv - kv0 - BN, D_v, D_v, tid);
        }

        if (wave_live && (!causal || kv0 <= wave_last_q)) {
            floatx16 sacc = floatx16{};
#pragma unroll
            for (int u = 0; u < HQ / 4; ++u) {
                const floatx4 kk = *reinterpret_cast<const floatx4*>(Ks + l32 * KS + HQ * hh + 4 * u);
#pragma unroll
                for (int e = 0; e < 4; ++e) sacc = mfma_f32(kk[e], qf[4 * u + e], sacc);
            }
            const bool need_mask = (kv0 + BN > S_kv) || (causal && kv0 + BN - 1 > qw0);
            float mx = -INFINITY;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                float x = sacc[r] * sl2;
                if (need_mask) {
                    const int key = kv0 + 8 * (r >> 2) + 4 * hh + (r & 3);
                    if (key >= S_kv || (causal && key > my_q)) x = -INFINITY;
                }
                sacc[r] = x;
                mx = fmaxf(mx, x);
            }
            mx = xhalf_max(mx);
            const float m_new = fmaxf(m_run, mx);
            if (wave_any(m_new > m_run + kTau)) {
                const float alpha = fast_exp2(m_run - m_new);
                l_run *= alpha;
#pragma unroll
                for (int dt = 0; dt < DV / 32; ++dt)
#pragma unroll
                    for (int r = 0; r < 16; ++r) oacc[dt][r] *= alpha;
                m_run = m_new;
            }
            const uint64_t st_blk = DROP ? st_base + (uint64_t)kv0 * kLcgMul : 0;
            float lsum = 0.f;
            float pr[16];
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                float pv = fast_exp2(sacc[r] - m_run);
                lsum += pv;
                if constexpr (DROP) {
                    const uint64_t off = (uint64_t)(8 * (r >> 2) + (r & 3)) * kLcgMul;
                    pv = lcg_keep(st_blk + off, thr) ? pv : 0.f;
                }
                pr[r] = pv;
            }
            l_run += lsum;
            // O^T += V^T P~^T: k-step r pairs lane-half h with key 8(r/4)+4h+r%4.
#pragma unroll
            for (int r = 0; r < 16; ++r) {
#pragma unroll
                for (int dt = 0; dt < DV / 32; ++dt) {
                    const float a = Vs[(8 * (r >> 2) + 4 * hh + (r & 3)) * VS + 32 * dt + l32];
                    oacc[dt] = mfma_f32(a, pr[r], oacc[dt]);
                }
            }
        }

        if (has_next) {
            float* Kn = lds + ((blk + 1) & 1) * Cfg::STAGE;
            kst.template store<KS>(Kn, tid);
            vst.template store<VS>(Kn + Cfg::KT, tid);
        }
        __syncthreads();
    }

    const float l_tot = xhalf_sum(l_run);
    if (my_q < S_q) {
        const float m_nat = (l_tot > 0.f) ? m_run * kLn2 : kNegInf;
        if (hh == 0) p.stats[(size_t)b * S_q + my_q] = m_nat + logf(l_tot + kEps);
        const float inv = (l_tot > kEps) ? p.c.keep_scale / l_tot : 0.f;
        float* Ob = static_cast<float*>(p.o) + ((size_t)b * S_q + my_q) * D_v;
#pragma unroll
        for (int dt = 0; dt < DV / 32; ++dt) {
#pragma unroll
            for (int g4 = 0; g4 < 4; ++g4) {
                const int d0 = 32 * dt + 8 * g4 + 4 * hh;
                floatx4 fv;
#pragma unroll
                for (int e = 0; e < 4; ++e) fv[e] = oacc[dt][4 * g4 + e] * inv;
                if constexpr (VEC) {
                    if (d0 < D_v) *reinterpret_cast<floatx4*>(Ob + d0) = fv;
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (d0 + e < D_v) Ob[d0 + e] = fv[e];
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Host launcher
// ---------------------------------------------------------------------------
hipError_t launch_fwd(const FwdParams& p, DType dtype, bool vec, hipStream_t stream) {
    const int B = p.s.B, S_q = p.s.S_q;
    if (B == 0 || S_q == 0) return hipSuccess;
    const bool drop = p.c.use_dropout != 0;
    return with_dim(p.s.D_qk, [&](auto dqk) {
        return with_dim(p.s.D_v, [&](auto dv) {
            return with_bool(vec, [&](auto v) {
                return with_bool(drop, [&](auto d) {
                    constexpr int DQK = decltype(dqk)::value, DV = decltype(dv)::value;
                    constexpr bool V = decltype(v)::value, D = decltype(d)::value;
                    if (dtype == DType::F16) {
                        using Cfg = FwdF16Cfg<DQK, DV>;
                        const int tiles = (S_q + Cfg::BM - 1) / Cfg::BM;
                        return launch_kernel<sdpa_fwd_f16_kernel<DQK, DV, V, D>>((unsigned)(tiles * B), Cfg::NT,
                                                                           Cfg::LDS_BYTES, stream, p);
                    } else {
                        using Cfg = FwdF32Cfg<DQK, DV>;
                        const int tiles = (S_q + Cfg::BM - 1) / Cfg::BM;
                        return launch_kernel<sdpa_fwd_f32_kernel<DQK, DV, V, D>>((unsigned)(tiles * B), Cfg::NT,
                                                                           Cfg::LDS_BYTES, stream, p);
                    }
                });
            });
        });
    });
}

}  // namespace sdpa
