// tile_order.hip -- CPU checks of the work order of the fp16 DMA kernels
// (xcd_map and row_window in sdpa_dma.h), built and run by
// tests/test_tile_order.py.  No GPU call: xcd_map runs on the host.
//
// With lin(b, t) = b * tiles + rank, rank = tiles-1-t when reversed (else t),
// for every (B, tiles, row bytes, reverse) of a grid:
//   - row_window(row bytes) = max(1, 8 MiB / row bytes);
//   - workgroup ids 0 .. B*tiles-1 map one to one onto (batch, tile);
//   - ids are dealt to XCDs as id % 8, and XCD x covers exactly the x-th of
//     8 contiguous lin ranges, whose lengths (nblocks / 8, the first
//     nblocks % 8 of them one longer) follow XCD order;
//   - in its dispatch order (id / 8 increasing) an XCD runs ceil(n / (wcap
//     tiles)) chunks of equal length (+-1, longer ones first) for its n ids;
//     each chunk covers a contiguous lin range, the chunks advance through
//     the XCD's range, and inside a chunk (rank, row) strictly increases;
//   - with B a multiple of 8 and wcap dividing B / 8 (the c3 and c4 cases),
//     every chunk is exactly wcap whole rows.
#include <cstdio>
#include <set>
#include <vector>

#include "sdpa_dma.h"

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

int main() {
    const size_t kCap = (size_t)8 << 20;
    const int Bs[] = {1, 2, 3, 7, 8, 9, 12, 16, 20, 24, 36, 40, 56, 64, 100, 128, 136, 256};
    const int Ts[] = {1, 2, 3, 4, 5, 6, 7, 8, 16, 32, 40};
    const int Ws[] = {1, 2, 3, 4, 5, 7, 16, 42, 1 << 20};  // chunk caps (row_window values)
    const size_t RB[] = {1024, (size_t)128 << 10, (size_t)512 << 10, (size_t)2 << 20, (size_t)3 << 20,
                         (size_t)9 << 20};
    int cases = 0;
    for (size_t rb : RB) {
        const int w = sdpa::row_window(rb);
        CHECK(w == (int)(kCap / rb > 0 ? kCap / rb : 1), "rb=%zu wcap=%d", rb, w);
    }
    for (int B : Bs)
        for (int wcap : Ws) {
            for (int T : Ts)
                for (int rev = 0; rev < 2; ++rev) {
                    ++cases;
                    const int n = B * T;
                    std::vector<int> seen((size_t)n, 0);
                    std::vector<std::vector<int>> lx(8);  // per XCD: lin values in dispatch order
                    for (int bid = 0; bid < n; ++bid) {
                        int b = -1, t = -1;
                        sdpa::xcd_map(bid, n, T, rev != 0, wcap, b, t);
                        CHECK(b >= 0 && b < B && t >= 0 && t < T, "B=%d T=%d bid=%d -> (%d,%d)", B, T, bid, b, t);
                        if (b < 0 || b >= B || t < 0 || t >= T) continue;
                        ++seen[(size_t)b * T + t];
                        lx[bid & 7].push_back(b * T + (rev ? T - 1 - t : t));
                    }
                    for (int i = 0; i < n; ++i) CHECK(seen[i] == 1, "B=%d T=%d tile %d seen %d", B, T, i, seen[i]);
                    int s_x = 0;
                    for (int x = 0; x < 8; ++x) {
                        const int n_x = n / 8 + (x < n % 8 ? 1 : 0);
                        CHECK((int)lx[x].size() == n_x, "B=%d T=%d xcd %d has %zu ids", B, T, x, lx[x].size());
                        if ((int)lx[x].size() != n_x) continue;
                        const std::set<int> lins(lx[x].begin(), lx[x].end());
                        CHECK(n_x == 0 || (*lins.begin() == s_x && *lins.rbegin() == s_x + n_x - 1 &&
                                           (int)lins.size() == n_x),
                              "B=%d T=%d xcd %d range", B, T, x);
                        if (n_x > 0) {
                            const int nch = (n_x + wcap * T - 1) / (wcap * T);
                            const int base = n_x / nch, extra = n_x % nch;
                            int pos = 0, prev_hi = s_x - 1;
                            for (int j = 0; j < nch; ++j) {
                                const int len = base + (j < extra ? 1 : 0);
                                int lo = lx[x][pos], hi = lx[x][pos];
                                for (int i = pos; i < pos + len; ++i) {
                                    lo = lx[x][i] < lo ? lx[x][i] : lo;
                                    hi = lx[x][i] > hi ? lx[x][i] : hi;
                                    if (i > pos) {
                                        const int r_a = lx[x][i - 1] % T, r_b = lx[x][i] % T;
                                        const int w_a = lx[x][i - 1] / T, w_b = lx[x][i] / T;
                                        CHECK(r_b > r_a || (r_b == r_a && w_b > w_a),
                                              "B=%d T=%d wcap=%d xcd %d chunk %d pos %d not rank-major", B, T, wcap, x, j, i);
                                    }
                                }
                                CHECK(hi - lo + 1 == len && lo == prev_hi + 1,
                                      "B=%d T=%d wcap=%d xcd %d chunk %d [%d,%d] len %d", B, T, wcap, x, j, lo, hi, len);
                                if (B % 8 == 0 && (B / 8) % wcap == 0)
                                    CHECK(len == wcap * T && lo % T == 0, "B=%d T=%d wcap=%d chunk not whole rows", B, T, wcap);
                                prev_hi = hi;
                                pos += len;
                            }
                        }
                        s_x += n_x;
                    }
                }
        }
    // wcap * tiles beyond 2^31 (dK/dV: a one-row query side against a long key
    // side gives a huge cap and many key tiles)
    for (int B : {1, 3, 9})
        for (int T : {8192, 20000}) {
            ++cases;
            const int n = B * T;
            std::vector<int> seen((size_t)n, 0);
            for (int bid = 0; bid < n; ++bid) {
                int b = -1, t = -1;
                sdpa::xcd_map(bid, n, T, false, 1 << 20, b, t);
                const bool ok = b >= 0 && b < B && t >= 0 && t < T;
                CHECK(ok, "huge cap B=%d T=%d bid=%d -> (%d,%d)", B, T, bid, b, t);
                if (ok) ++seen[(size_t)b * T + t];
            }
            for (int i = 0; i < n; ++i) CHECK(seen[i] == 1, "huge cap B=%d T=%d tile %d seen %d", B, T, i, seen[i]);
        }
    if (fails) {
        std::printf("%d failures over %d cases\n", fails, cases);
        return 1;
    }
    std::printf("ok %d cases\n", cases);
    return 0;
}
