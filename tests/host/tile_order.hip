// tile_order.hip -- CPU checks of the work order of the fp16 DMA kernels
// (xcd_map and row_window in sdpa_dma.h), built and run by
// tests/test_tile_order.py.  No GPU call: xcd_map runs on the host.
//
// For every (B, tiles, row bytes, reverse) of a grid:
//   - row_window is 1 when B is not a multiple of 8, else the largest divisor
//     of B / 8 whose rows stream at most 8 MiB (1 if none);
//   - workgroup ids 0 .. B*tiles-1 map one to one onto (batch, tile);
//   - ids are dealt to XCDs as id % 8; with B a multiple of 8, XCD x gets
//     exactly the batch rows [x B/8, (x+1) B/8);
//   - in each XCD's dispatch order (id / 8 increasing), the windows of rows
//     come one after another, and inside a window the tiles run by rank
//     (rank = tiles-1-t when reversed, else t) with every row of the window
//     taking rank r before any row takes rank r+1.
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
    const int Bs[] = {1, 2, 3, 7, 8, 9, 16, 24, 40, 64, 128, 136, 256};
    const int Ts[] = {1, 2, 3, 5, 16, 32};
    const size_t RB[] = {1024, (size_t)128 << 10, (size_t)512 << 10, (size_t)2 << 20, (size_t)3 << 20,
                         (size_t)9 << 20};
    int cases = 0;
    for (int B : Bs)
        for (size_t rb : RB) {
            const int win = sdpa::row_window(B, rb);
            if (B % 8) {
                CHECK(win == 1, "B=%d rb=%zu win=%d", B, rb, win);
            } else {
                const int rows = B / 8;
                CHECK(win >= 1 && rows % win == 0, "B=%d rb=%zu win=%d", B, rb, win);
                CHECK(win == 1 || (size_t)win * rb <= kCap, "B=%d rb=%zu win=%d", B, rb, win);
                for (int d = win + 1; d <= rows; ++d)
                    CHECK(rows % d != 0 || (size_t)d * rb > kCap, "B=%d rb=%zu win=%d d=%d", B, rb, win, d);
            }
            for (int T : Ts)
                for (int rev = 0; rev < 2; ++rev) {
                    ++cases;
                    const int n = B * T;
                    std::vector<int> seen((size_t)n, 0);
                    std::vector<std::vector<int>> bx(8), rx(8);  // per XCD, in dispatch order
                    for (int bid = 0; bid < n; ++bid) {
                        int b = -1, t = -1;
                        sdpa::xcd_map(bid, n, T, rev != 0, win, b, t);
                        CHECK(b >= 0 && b < B && t >= 0 && t < T, "B=%d T=%d bid=%d -> (%d,%d)", B, T, bid, b, t);
                        if (b < 0 || b >= B || t < 0 || t >= T) continue;
                        ++seen[(size_t)b * T + t];
                        bx[bid & 7].push_back(b);
                        rx[bid & 7].push_back(rev ? T - 1 - t : t);
                    }
                    for (int i = 0; i < n; ++i) CHECK(seen[i] == 1, "B=%d T=%d tile %d seen %d", B, T, i, seen[i]);
                    for (int x = 0; x < 8; ++x) {
                        if (B % 8 == 0) {
                            const std::set<int> rows(bx[x].begin(), bx[x].end());
                            const int lo = x * (B / 8), hi = (x + 1) * (B / 8);
                            CHECK((int)rows.size() == B / 8 && *rows.begin() == lo && *rows.rbegin() == hi - 1,
                                  "B=%d T=%d xcd %d rows %zu", B, T, x, rows.size());
                        }
                        // windows in order; inside one, rank-major over its rows
                        for (size_t i = 1; i < bx[x].size(); ++i) {
                            const int g0 = bx[x][i - 1] / win, g1 = bx[x][i] / win;
                            CHECK(g1 >= g0, "B=%d T=%d xcd %d window order", B, T, x);
                            if (g1 == g0)
                                CHECK(rx[x][i] > rx[x][i - 1] || (rx[x][i] == rx[x][i - 1] && bx[x][i] > bx[x][i - 1]),
                                      "B=%d T=%d win=%d xcd %d pos %zu", B, T, win, x, i);
                        }
                    }
                }
        }
    if (fails) {
        std::printf("%d failures over %d cases\n", fails, cases);
        return 1;
    }
    std::printf("ok %d cases\n", cases);
    return 0;
}
