// Host-side checks of the work orders that the kernels and launchers share
// (mx230_amd/csrc/fa_device.h), under AddressSanitizer and
// UndefinedBehaviorSanitizer; nothing touches a device. Exit status 0 = all
// checks passed.
//  * cu_order_wg: a permutation of the work-group indices; and, under the
//    dispatcher model (work-group i on XCD i mod 8, then round robin over
//    that XCD's CUs, so i and i + 256 share a CU), the resident work-groups of
//    a causal launch (heaviest first, heads fastest) give every CU the same
//    stages up to one per pair of runs of 256 and two for a triple (an odd
//    count of runs), the rounding of each block's stages to its rank.
//  * dkv_first_work: share 0 of each (batch, KV head, key block) is the
//    dkv_work index whose work is that block's share 0, and the block's shares
//    are the indices after it, for split and unsplit, causal and not.
#include <algorithm>
#include <cstdio>
#include <cstring>
#include <vector>

#include "../../mx230_amd/csrc/fa_device.h"

using namespace mxfa;

static int g_fail = 0;
#define CHECK(cond, ...)                                     \
    do {                                                     \
        if (!(cond)) {                                       \
            std::fprintf(stderr, "FAIL %s:%d: ", __FILE__, __LINE__); \
            std::fprintf(stderr, __VA_ARGS__);               \
            std::fputc('\n', stderr);                        \
            ++g_fail;                                        \
        }                                                    \
    } while (0)

static void check_cu_order() {
    // a permutation of [0, n) for every run length and count of runs inside n
    for (int n = 1; n <= 200; n += 7) {
        for (int run = 0; run <= n; run += 3) {
            for (int runs = 0; run > 0 && runs * run <= n; ++runs) {
                std::vector<int> seen(n, 0);
                for (int i = 0; i < n; ++i) {
                    const int r = cu_order_wg(i, run, runs);
                    CHECK(r >= 0 && r < n, "n %d run %d runs %d: %d -> %d", n, run, runs, i, r);
                    if (r >= 0 && r < n) ++seen[r];
                }
                for (int r = 0; r < n; ++r) CHECK(seen[r] == 1, "n %d run %d runs %d: rank %d seen %d times", n, run, runs, r, seen[r]);
            }
        }
    }
    // per-CU stages of the resident work-groups under the dispatcher model:
    // bh heads, nqb blocks, occ work-groups per CU (the kernel's occupancy);
    // the launcher balances the whole runs of 256 among the resident ones
    constexpr int C = 256;
    for (int bh : {8, 14, 28, 32, 48, 64, 96, 128}) {
        for (int nqb : {16, 24, 32, 48, 64}) {
            for (int occ : {2, 3, 4}) {
                const long long total = (long long)bh * nqb, resident = std::min<long long>(total, C * occ);
                const int runs = (int)(resident / C);
                if (runs < 2) continue;
                std::vector<long long> cu(C, 0), plain(C, 0);
                for (int i = 0; i < runs * C; ++i) {
                    const int xcd = i % 8, slot = (i / 8) % (C / 8);  // dispatch model
                    const int r = cu_order_wg(i, C, runs);
                    cu[xcd * (C / 8) + slot] += nqb - r / bh;    // stages of the rank's block (heaviest first)
                    plain[xcd * (C / 8) + slot] += nqb - i / bh;
                }
                const auto spread = [](const std::vector<long long> &v) {
                    long long lo = v[0], hi = v[0];
                    for (long long x : v) {
                        lo = x < lo ? x : lo;
                        hi = x > hi ? x : hi;
                    }
                    return hi - lo;
                };
                const long long bound = runs % 2 ? (runs - 3) / 2 + 2 : runs / 2;
                CHECK(spread(cu) <= bound, "bh %d nqb %d occ %d: per-CU stages spread %lld (bound %lld, plain order %lld)",
                      bh, nqb, occ, spread(cu), bound, spread(plain));
                CHECK(spread(cu) <= spread(plain), "bh %d nqb %d occ %d: balanced %lld against plain %lld", bh, nqb, occ,
                      spread(cu), spread(plain));
            }
        }
    }
}

static Params plan(int B, int Hkv, int group, int N, int split, int min_shares, int share_stages) {
    Params p;
    std::memset(&p, 0, sizeof(p));
    p.B = B;
    p.Hkv = Hkv;
    p.group = group;
    p.Hq = Hkv * group;
    p.N = N;
    p.dkv_split = split;
    p.dkv_min_shares = min_shares;
    p.dkv_share_stages = share_stages;
    return p;
}

static void check_first_work() {
    const int bkv_rows[] = {128, 64}, bq = 64;
    for (int rows : bkv_rows) {
        for (bool causal : {false, true}) {
            const Params plans[] = {
                plan(1, 4, 8, 2048, 1, 1, 1 << 30),   // unsplit
                plan(1, 4, 8, 2048, 2, 8, 17),        // cfg5-like: more shares for the heavy blocks
                plan(2, 2, 7, 4096, 2, 7, 58),        // cfg4-like
                plan(1, 2, 5, 836, 2, 5, 9),          // runs that start inside a head
                plan(3, 1, 16, 1000, 2, 2, 12),       // MQA-like, ragged
                plan(1, 2, 4, 77, 2, 4, 8),           // tiny
            };
            for (Params p : plans) {
                const int nkb = (p.N + rows - 1) / rows, nbkv = p.B * p.Hkv;
                if (p.dkv_split > 1) {  // as the planner does: dkv_split = the most shares of any block
                    int most = 1;
                    for (int kb = 0; kb < nkb; ++kb) {
                        const int s = dkv_block_shares(p, (p.N - (causal ? kb * rows : 0) + bq - 1) / bq);
                        most = s > most ? s : most;
                    }
                    p.dkv_split = most > 1 ? most : 2;
                }
                int total = 0;
                for (int kb = 0; kb < nkb; ++kb) {
                    total += nbkv * dkv_block_shares(p, (p.N - (causal ? kb * rows : 0) + bq - 1) / bq);
                }
                std::vector<int> seen(total, 0);
                for (int kb = 0; kb < nkb; ++kb) {
                    for (int bkv = 0; bkv < nbkv; ++bkv) {
                        const int ns = dkv_block_shares(p, (p.N - (causal ? kb * rows : 0) + bq - 1) / bq);
                        const int w0 = dkv_first_work(p, bkv, kb, rows, bq, causal);
                        for (int sp = 0; sp < ns; ++sp) {
                            const int w = w0 + sp;
                            CHECK(w >= 0 && w < total, "N %d kb %d bkv %d sp %d: index %d of %d", p.N, kb, bkv, sp, w,
                                  total);
                            if (w < 0 || w >= total) continue;
                            ++seen[w];
                            const DkvWork wk = dkv_work(p, w, rows, bq, causal);
                            CHECK(wk.bkv == bkv && wk.kb == kb && wk.sp == sp && wk.ns == ns,
                                  "N %d split %d causal %d rows %d: index %d is (%d, %d, %d/%d), want (%d, %d, %d/%d)",
                                  p.N, p.dkv_split, (int)causal, rows, w, wk.bkv, wk.kb, wk.sp, wk.ns, bkv, kb, sp, ns);
                        }
                    }
                }
                for (int w = 0; w < total; ++w) CHECK(seen[w] == 1, "N %d: index %d seen %d times", p.N, w, seen[w]);
                CHECK(dkv_work(p, total, rows, bq, causal).kb == nkb || p.dkv_split <= 1 || !causal,
                      "N %d: the index past the last share does not report the end", p.N);
            }
        }
    }
}

int main() {
    check_cu_order();
    check_first_work();
    if (g_fail != 0) {
        std::fprintf(stderr, "%d checks failed\n", g_fail);
        return 1;
    }
    std::printf("all checks passed\n");
    return 0;
}
