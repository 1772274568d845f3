// ds_layout.hip -- CPU checks of the stored-dS layouts of the backward's dS
// path (DsLayoutT, DsLayout::slot, DsLayout32::slot32 in sdpa_params.h), built
// and run by tests/test_ds_layout.py.  No GPU call.
//
// For both chunk walks (fp16: query blocks of 64, fp32: 32) over a grid of
// (S_q, S_kv, causal), with B = 2:
//   - prefix(kt) equals the count of the chunks the dK/dV kernel visits in
//     the key tiles before kt (its q_begin walk), and qbb(kt) its first block;
//   - every visited chunk has its own offset, inside bytes(B);
//   - every (key group, query block) the dQ kernel reads as live is a chunk
//     the dK/dV kernel wrote (fp16: 64-query waves of two 32-query sub-tiles,
//     fp32: 32-query waves; 32-key steps).
// Inside a chunk:
//   - fp16: slot(key, p) maps the 32 keys x 4 planes of a 2 KB key group one
//     to one onto its 16-byte slots, and store j of the 64 lanes (planes
//     2 j, 2 j + 1) fills the KB at 1024 j whole;
//   - fp32: slot32(key, pos) maps 32 keys x 32 positions one to one onto the
//     4-byte words of a 4 KB key group; store u of lane (h, key) is one 16-byte
//     slot holding positions 16 h + 4 u .. + 3 in order, and the 64 lanes of
//     store u fill the KB at 1024 u whole; the dQ kernel's read of key
//     2 p + hh at position l32 is slot32(2 (p & 3) + hh, l32) + 128 (p >> 2),
//     and its 32 lanes of one half-wave read 32 different 4-byte LDS banks.
#include <cstdio>
#include <set>
#include <vector>

#include "sdpa_params.h"

static int fails = 0;
#define CHECK(cond, ...)                             \
    do {                                             \
        if (!(cond)) {                               \
            if (fails++ < 20) {                      \
                std::printf("FAIL %s: ", #cond);     \
                std::printf(__VA_ARGS__);            \
                std::printf("\n");                   \
            }                                        \
        }                                            \
    } while (0)

template <int QBK>
static void check_walk(int S_q, int S_kv, bool causal) {
    using L = sdpa::DsLayoutT<QBK>;
    const L dsl(S_q, S_kv, causal);
    const int B = 2;
    long long acc = 0;
    std::set<size_t> offs;
    std::set<long long> written;  // (b, kt, qb) written by the dK/dV walk
    for (int kt = 0; kt <= dsl.tiles; ++kt) {
        CHECK(dsl.prefix(kt) == acc, "QBK %d S_q %d S_kv %d causal %d kt %d prefix %lld walk %lld", QBK, S_q, S_kv,
              (int)causal, kt, dsl.prefix(kt), acc);
        if (kt == dsl.tiles) break;
        const int k0 = 128 * kt;
        const int q_begin = causal ? ((k0 < S_q ? k0 : S_q) / QBK) * QBK : 0;
        const int nblk = (S_q - q_begin + QBK - 1) / QBK;
        CHECK(q_begin / QBK == dsl.qbb(kt), "QBK %d S_q %d kt %d qbb", QBK, S_q, kt);
        for (int b = 0; b < B; ++b)
            for (int m = 0; m < nblk; ++m) {
                const int qb = q_begin / QBK + m;
                const size_t off = dsl.offset(b, kt, qb);
                CHECK(off % L::CHUNK == 0 && off + L::CHUNK <= dsl.bytes(B), "offset in bounds");
                CHECK(offs.insert(off).second, "QBK %d S_q %d S_kv %d kt %d qb %d offset reused", QBK, S_q, S_kv, kt, qb);
                written.insert(((long long)b * 4096 + kt) * 4096 + qb);
            }
        acc += nblk;
    }
    // the dQ kernel's live (key group, query block) pairs
    const int QW = QBK == 64 ? 64 : 32;  // queries per dQ wave
    for (int b = 0; b < B; ++b)
        for (int qw0 = 0; qw0 < S_q; qw0 += QW) {
            const int qb = qw0 / QBK;
            for (int kv0 = 0; kv0 < S_kv; kv0 += 32) {
                bool live = false;
                for (int t = 0; t < QW / 32; ++t) {
                    const int qs = qw0 + 32 * t;
                    live |= qs < S_q && !(causal && qs + 31 < kv0);
                }
                if (!live) continue;
                CHECK(written.count(((long long)b * 4096 + kv0 / 128) * 4096 + qb) == 1,
                      "QBK %d S_q %d S_kv %d causal %d: dQ reads (kv0 %d, qb %d) the dK/dV kernel did not write", QBK,
                      S_q, S_kv, (int)causal, kv0, qb);
            }
        }
}

static void check_slots() {
    // fp16 planes
    std::set<int> s16;
    for (int p = 0; p < 4; ++p)
        for (int key = 0; key < 32; ++key) {
            const int o = sdpa::DsLayout::slot(key, p);
            CHECK(o % 16 == 0 && o >= 0 && o < 2048, "fp16 slot range");
            s16.insert(o);
        }
    CHECK(s16.size() == 128, "fp16 slots one to one");
    for (int j = 0; j < 2; ++j) {
        std::set<int> kb;
        for (int h = 0; h < 2; ++h)
            for (int key = 0; key < 32; ++key) kb.insert(sdpa::DsLayout::slot(key, 2 * j + h));
        CHECK(kb.size() == 64 && *kb.begin() == 1024 * j && *kb.rbegin() == 1024 * j + 1008, "fp16 store %d one KB", j);
    }
    // fp32 slots
    std::set<int> s32;
    for (int key = 0; key < 32; ++key)
        for (int pos = 0; pos < 32; ++pos) {
            const int o = sdpa::DsLayout32::slot32(key, pos);
            CHECK(o % 4 == 0 && o >= 0 && o < 4096, "fp32 slot range");
            s32.insert(o);
        }
    CHECK(s32.size() == 1024, "fp32 slots one to one");
    for (int u = 0; u < 4; ++u) {
        std::set<int> kb;
        for (int h = 0; h < 2; ++h)
            for (int key = 0; key < 32; ++key) {
                const int a = sdpa::DsLayout32::slot32(key, 16 * h + 4 * u);
                CHECK(a % 16 == 0, "fp32 store slot aligned");
                for (int e = 0; e < 4; ++e)
                    CHECK(sdpa::DsLayout32::slot32(key, 16 * h + 4 * u + e) == a + 4 * e, "fp32 positions in order");
                kb.insert(a);
            }
        CHECK(kb.size() == 64 && *kb.begin() == 1024 * u && *kb.rbegin() == 1024 * u + 1008, "fp32 store %d one KB", u);
    }
    for (int hh = 0; hh < 2; ++hh)
        for (int pr = 0; pr < 16; ++pr) {
            std::set<int> banks;
            for (int l32 = 0; l32 < 32; ++l32) {
                const int a = sdpa::DsLayout32::slot32(2 * pr + hh, l32);
                CHECK(a == sdpa::DsLayout32::slot32(2 * (pr & 3) + hh, l32) + 128 * (pr >> 2), "fp32 reader base + immediate");
                banks.insert((a / 4) % 64);
            }
            CHECK(banks.size() == 32, "fp32 reader banks, key pair %d hh %d", pr, hh);
        }
}

int main() {
    const int sq[] = {1, 31, 32, 33, 63, 64, 65, 127, 128, 129, 200, 256, 333, 512, 1000, 1024, 4096};
    const int skv[] = {1, 32, 100, 127, 128, 129, 300, 1000, 4096};
    for (int S_q : sq)
        for (int S_kv : skv)
            for (int c = 0; c < 2; ++c) {
                if (c && S_q != S_kv) continue;  // the op rejects a causal mask over unequal lengths
                check_walk<64>(S_q, S_kv, c != 0);
                check_walk<32>(S_q, S_kv, c != 0);
            }
    for (int S : {1, 5, 100, 200, 333, 1000})
        for (int c = 0; c < 2; ++c) {
            check_walk<64>(S, S, c != 0);
            check_walk<32>(S, S, c != 0);
        }
    check_slots();
    if (fails) {
        std::printf("%d failures\n", fails);
        return 1;
    }
    std::printf("ok\n");
    return 0;
}
