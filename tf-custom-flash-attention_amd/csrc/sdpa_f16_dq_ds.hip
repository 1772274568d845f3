// sdpa_f16_dq_ds.hip -- the dS path of the fp16 SdpaGrad for gfx950: dQ as a
// product with the dS' the dK/dV kernel stored, instead of a kernel that
// forms S, P, dP and dS once more.
//
// Order of the path (sdpa_capi.hip):
//   1. row kernel  -- stats2 and delta per query row into the workspace (the
//                     values the dQ kernel of the other path writes first);
//   2. dK/dV       -- the split-role kernel (sdpa_f16_dkdv_split.hip) with
//                     p.ds set: its dS role stores every dS' it forms;
//   3. dQ          -- dQ^T = K^T dS'^T per 32 queries, scaled once at the store.
// dQ then costs one fp16 read of dS' (2 bytes per visited score) instead of
// three products and the element-wise work per score; the dS' it reads are
// the ones dK was formed from.
//
// Element semantics (sdpa/sdpa_bwd.cu.cc:291-327): dQ_i = scale sum_j dS_ij
// K_j, with dS as the dK/dV kernel forms it (P from the fp16 P of its P role,
// the 1e-6 gate, the dropout decision; with dropout dS' = dS (1-p), scaled
// back by 1/(1-p) at the store).
#include <type_traits>

#include "sdpa_dma.h"
#include "sdpa_launch.h"
#include "sdpa_params.h"

namespace sdpa {
namespace {

// ---------------------------------------------------------------------------
// Row values.  One lane pair per query row (lane = row, hh = half of the
// features): delta = sum_d dO O in the order of the dQ kernel's prologue, and
// stats2 = stats log2(e) + kGateShift as one fma, so that both paths hand the
// dK/dV kernel the same values.  The 128 rows of dO and O a workgroup covers
// are first copied into LDS whole (each copy 1 KB of consecutive bytes; a
// lane's own 16-byte pieces, 32 rows apart per load, made every lane a
// request of its own) and read back per lane in the swizzled row layout.
// ---------------------------------------------------------------------------
template <int DV>
struct RowsCfg {
    static constexpr int NW = 4, NT = 64 * NW, ROWS = 32 * NW, L = DV / 8;
    static constexpr int TB = ROWS * L * 16;  // one tile (dO or O)
    static constexpr size_t LDS_BYTES = 2 * (size_t)TB;
};

template <int DV>
__global__ __launch_bounds__(256) void sdpa_bwd_rows_f16_kernel(const BwdParams p) {
    using Cfg = RowsCfg<DV>;
    constexpr int L = Cfg::L, ROWS = Cfg::ROWS, NW = Cfg::NW, TB = Cfg::TB;
    const int tid = threadIdx.x, lane = tid & 63, l32 = lane & 31, hh = lane >> 5;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int S_q = p.s.S_q, D_v = p.s.D_v;
    const int tiles = (S_q + ROWS - 1) / ROWS;
    const int b = (int)(blockIdx.x / (unsigned)tiles), qt = (int)(blockIdx.x % (unsigned)tiles);
    const int q0 = qt * ROWS, my_q = q0 + 32 * wave + l32;
    const size_t row0 = (size_t)b * S_q + q0;
    // rows past S_q and features past D_v read as zero
    TileCopy<ROWS, L, NW> tc;
    tc.init(wave, lane, D_v * 2, D_v / 8);
    const uint32_t m0 = lds_base() + 1024u * (uint32_t)wave;
    tc.issue(row_src(p.d_o, row0, S_q - q0, D_v * 2), m0, wave);
    tc.issue(row_src(p.o, row0, S_q - q0, D_v * 2), m0 + (uint32_t)TB, wave);
    wait_vm();
    __syncthreads();
    SwzLane<L> sw;
    sw.init(lane);
    float dpart = 0.f;
#pragma unroll
    for (int ks = 0; ks < DV / 16; ++ks) {
        const half8 d8 = lds_row<L>(sw.row, ks, 32 * wave);
        const half8 o8 = lds_row<L>(TB + sw.row, ks, 32 * wave);
#pragma unroll
        for (int e = 0; e < 8; ++e) dpart += (float)d8[e] * (float)o8[e];
    }
    const float delta = xhalf_sum(dpart);
    if (my_q < S_q && hh == 0) {
        const size_t row_q = (size_t)b * S_q + my_q;
        p.delta[row_q] = delta;
        p.stats2[row_q] = __builtin_fmaf(p.stats[row_q], kLog2e, kGateShift);
    }
}

// ---------------------------------------------------------------------------
// dQ from the stored dS'.  Four waves of 64 queries (256 per workgroup): a
// wave owns one stored query block (its two 32-query sub-tiles), so every
// K^T operand it reads from LDS feeds two MFMAs.  Key steps of 32 (one stored
// key group) through a three-stage LDS ring of the K tile (read transposed:
// the A operand K^T) and each wave's two dS' tiles, 32 keys x 32 queries as
// stored (read transposed: the B operand dS'^T, lane = query).  The lanes of
// a wave take the queries in the stored order (DsLayout), so the tiles are
// copied as they lie (2 KB each, lane-contiguous); lane l32 owns queries
// qb 64 + 32 t + pi(l32).
// ---------------------------------------------------------------------------
template <int DQK>
struct DqDsCfg {
    static constexpr int NW = 4, NT = 64 * NW, BM = 64 * NW, BN = 32, NSTAGE = 3;
    static constexpr int LK = DQK / 8;
    static constexpr int KB = BN * DQK * 2;  // K tile
    static constexpr int SB = BN * 64;       // one 32-query dS' tile
    static constexpr int STAGE = KB + 2 * NW * SB;
    static constexpr size_t LDS_BYTES = NSTAGE * (size_t)STAGE;
    static_assert(2 * LDS_BYTES <= 160 * 1024, "two workgroups per CU");
};

template <int DQK, bool CAUSAL>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2)))
void sdpa_bwd_dq_ds_f16_kernel(const BwdParams p, const int win) {
    using Cfg = DqDsCfg<DQK>;
    constexpr int BM = Cfg::BM, BN = Cfg::BN, LK = Cfg::LK, NW = Cfg::NW, NSTAGE = Cfg::NSTAGE, NDT = DQK / 32;
    static_assert(DsLayout::KT % BN == 0 && BM % DsLayout::QBK == 0, "steps tile the stored chunks");

    const int tid = threadIdx.x, lane = tid & 63, l32 = lane & 31, hh = lane >> 5;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int B = p.s.B, S_q = p.s.S_q, S_kv = p.s.S_kv, D_qk = p.s.D_qk;
    const int tiles = (S_q + BM - 1) / BM;
    int b, qt;
    xcd_map(blockIdx.x, B * tiles, tiles, CAUSAL, win, b, qt);
    const int q0 = qt * BM, qw0 = q0 + 64 * wave, qb = qw0 / DsLayout::QBK;
    const int pq = 8 * ((l32 >> 2) & 3) + 4 * (l32 >> 4) + (l32 & 3);  // stored position -> query
    const DsLayout dsl(S_q, S_kv, CAUSAL);
    const unsigned char* dsb = static_cast<const unsigned char*>(p.ds);

    // Sub-tile t (queries qw0 + 32 t ..) at the key group kv0: stored by the
    // dK/dV kernel under the same predicate (its sub_live), and then in a
    // visited chunk (keys from kt 128 up to query qw0 + 32 t + 31 put the
    // query block at or past qbb(kt)).  Under the causal mask either may be
    // live without the other (the group at qw0 + 32 reaches sub-tile 1 only).
    auto sub_live = [&](int kv0, int t) {
        const int qs = qw0 + 32 * t;
        return qs < S_q && kv0 < S_kv && !(CAUSAL && qs + 31 < kv0);
    };

    const RowSrc ksrc = row_src(p.k, (size_t)b * S_kv, S_kv, D_qk * 2);
    TileCopy<BN, LK, NW, true> kc;
    kc.init(wave, lane, D_qk * 2, D_qk / 8);
    TileCopy<BN, 4, 1, true> sc;  // lane offsets of a plain 2 KB copy (32 rows of 64 bytes)
    sc.init(0, lane, 64, 4);
    const uint32_t lds0 = lds_base();
    const int kv_end = CAUSAL ? min(S_kv, q0 + BM) : S_kv;
    const int nsteps = (kv_end + BN - 1) / BN;
    // Copies of step `step` into stage step % NSTAGE: the wave's share of the
    // K tile and its live dS' tiles.  Returns the number of copies issued.
    auto issue = [&](int step) {
        const int kv0 = step * BN;
        const uint32_t so = (uint32_t)((step % NSTAGE) * Cfg::STAGE);
        kc.issue(ksrc.shifted(kv0), lds0 + so + 1024u * (uint32_t)wave, wave);
        int n = decltype(kc)::count(wave);
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            if (sub_live(kv0, t)) {
                const unsigned char* src = dsb + dsl.offset(b, kv0 / DsLayout::KT, qb) + t * 8192 +
                                           (kv0 % DsLayout::KT) * 64;
                // dS is read once: non-temporal (dQ 0.470 -> 0.425 ms at c4)
                const rsrc_t rs = RowSrc{uniform_ptr(src), BN, 64, 0x7FFFFFFF / 64}.at(0);
                const uint32_t m0 = lds0 + so + (uint32_t)(Cfg::KB + Cfg::SB * (2 * wave + t));
#pragma unroll
                for (int u = 0; u < decltype(sc)::count(0); ++u) dma16_at_nt(rs, m0 + 1024u * u, sc.voff + 1024u * u);
                n += decltype(sc)::count(0);
            }
        }
        return n;
    };

    floatx16 acc[2][NDT];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) acc[t][dt] = floatx16{};
    const uint32_t kl = lds0 + tr_lane_off<LK>(lane);                                           // K^T
    // dS'^T: the transposed read of tr_lane_off<4> (row tr_row, 16-byte slot
    // c: query positions 8 c + sub / 2 ..) at its place in the stored tile,
    // slot(key, p) with p = 2 (c & 1) + (c >> 1); rows tr_row and tr_row + 8
    // (slot(key + 16 n, p) = slot(key, p) + 256 n)
    uint32_t sl0, sl8;
    {
        const int g16 = lane >> 4, i16 = lane & 15;
        const int tr_row = 4 * (g16 >> 1) + (i16 >> 2), c = 2 * (g16 & 1) + ((i16 & 3) >> 1), sub = 8 * (i16 & 1);
        const int pl = 2 * (c & 1) + (c >> 1);
        const uint32_t base = lds0 + (uint32_t)(Cfg::KB + Cfg::SB * 2 * wave + sub);
        sl0 = base + (uint32_t)DsLayout::slot(tr_row, pl);
        sl8 = base + (uint32_t)DsLayout::slot(tr_row + 8, pl);
    }

    // One key step: two 16-key halves.  Element i of a transposed read (two
    // ds_read_b64_tr_b16 of four rows each) holds row R0 + 8 (i / 4) + 4 hh +
    // i % 4, for the K^T and the dS'^T operand alike.  Keys past S_kv need no
    // mask: their K rows read as zero and the dK/dV kernel stored a zero dS'
    // for them.  A sub-tile that is not live (its queries all before the key
    // group, or past S_q) takes a zero operand instead of its stale tile.
    auto step_mfma = [&](uint32_t so, bool t0, bool t1) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int R0 = 16 * j;
            half8 bs[2];
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                const uint32_t a = so + (uint32_t)(Cfg::SB * t) + 16u * R0;
                bs[t] = ld_tr8(sl0 + a, sl8 + a);
            }
            if (!t0) bs[0] = half8{};
            if (!t1) bs[1] = half8{};
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt) {
                const uint32_t a = (kl ^ (uint32_t)(64 * dt)) + so;
                const half8 ak = ld_tr8(a + 16u * LK * R0, a + 16u * LK * (R0 + 8));
#pragma unroll
                for (int t = 0; t < 2; ++t) acc[t][dt] = mfma_f16(ak, bs[t], acc[t][dt]);
            }
        }
    };

    // Ring: the copies of step n + 2 go out once step n begins (their stage
    // held step n - 1, which every wave has finished at that barrier); step
    // n waits for its own copies with those of step n + 1 still in flight.
    static_assert(NSTAGE == 3, "two steps of copies ahead");
    int n_next = 0;  // copies of step n + 1 this wave issued
    if (nsteps > 0) issue(0);
    if (nsteps > 1) n_next = issue(1);
    for (int step = 0; step < nsteps; ++step) {
        if (step + 1 < nsteps) wait_vm_upto(n_next);
        else wait_vm();
        __syncthreads();
        if (step + 2 < nsteps) n_next = issue(step + 2);
        else n_next = 0;
        const int kv0 = step * BN;
        const bool t0 = sub_live(kv0, 0), t1 = sub_live(kv0, 1);
        if (t0 || t1) step_mfma((uint32_t)((step % NSTAGE) * Cfg::STAGE), t0, t1);
    }

    // dS' = dS (1-p) with dropout (keep_scale 1/(1-p)); every element
    // dropped (keep_scale 0): dS' = dS
    const float f = (p.c.use_dropout && p.c.keep_scale != 0.f) ? p.c.scale * p.c.keep_scale : p.c.scale;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        const int my_q = qw0 + 32 * t + pq;
        if (my_q < S_q) {
            half_t* dQb = static_cast<half_t*>(p.dq) + ((size_t)b * S_q + my_q) * D_qk;
            if (D_qk == DQK) store_rows_f16<DQK>(dQb, acc[t], f, hh);
            else store_rows_f16_n<DQK>(dQb, acc[t], f, hh, D_qk);
        }
    }
}

}  // namespace

hipError_t launch_bwd_rows_f16(const BwdParams& p, hipStream_t stream) {
    const int B = p.s.B, S_q = p.s.S_q;
    if (B == 0 || S_q == 0) return hipSuccess;
    const long long n = (long long)((S_q + 127) / 128) * B;
    if (n > 0x7FFFFFFFLL) return hipErrorInvalidValue;
    return with_dim(p.s.D_v, [&](auto dv) {
        constexpr int DV = decltype(dv)::value;
        using Cfg = RowsCfg<DV>;
        return launch_kernel<sdpa_bwd_rows_f16_kernel<DV>>((unsigned)n, Cfg::NT, Cfg::LDS_BYTES, stream, p);
    });
}

hipError_t launch_bwd_dq_ds_f16(const BwdParams& p, hipStream_t stream) {
    const int B = p.s.B, S_q = p.s.S_q;
    if (B == 0 || S_q == 0) return hipSuccess;
    if (!p.ds) return hipErrorInvalidValue;
    return with_dim(p.s.D_qk, [&](auto dqk) {
        return with_bool(p.c.causal != 0, [&](auto c) {
            constexpr int DQK = decltype(dqk)::value;
            using Cfg = DqDsCfg<DQK>;
            const long long n = (long long)((S_q + Cfg::BM - 1) / Cfg::BM) * B;
            return launch_kernel<sdpa_bwd_dq_ds_f16_kernel<DQK, decltype(c)::value>>(
                (unsigned)n, Cfg::NT, Cfg::LDS_BYTES, stream, p, row_window((size_t)p.s.S_kv * DQK * 2));
        });
    });
}

}  // namespace sdpa
