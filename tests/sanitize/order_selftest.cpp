// Host-side checks of the work orders that the kernels and launchers share
// (mx230_amd/csrc/fa_device.h), under AddressSanitizer and
// UndefinedBehaviorSanitizer; nothing touches a device. Exit status 0 = all
// checks passed.
//  * cu_order_block: a permutation of the block indices whenever the period
//    divides their count; and, for a causal grid resident all at once that
//    the dispatcher places work-group i on XCD i mod 8 and, within the XCD,
//    round robin over its 32 CUs, every CU gets the same number of stages
//    when the runs of `period` blocks pair up (an even count of them), and
//    stages within period - 1 of each other otherwise (the last run alone),
//    where the plain order spreads them by (runs) x (period - 1).
//  * dkv_first_work: share 0 of each (batch, KV head, key block) is the
//    dkv_work index whose work is that block's share 0, and the block's shares
//    are the indices after it, for split and unsplit, causal and not.
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
    // a permutation for every period that divides the count
    for (int n = 1; n <= 96; ++n) {
        for (int period = 0; period <= n; ++period) {
            if (period > 1 && n % period != 0) continue;
            std::vector<int> seen(n, 0);
            for (int y = 0; y < n; ++y) {
                const int b = cu_order_block(y, period);
                CHECK(b >= 0 && b < n, "n %d period %d: y %d -> %d", n, period, y, b);
                if (b >= 0 && b < n) ++seen[b];
            }
            for (int b = 0; b < n; ++b) CHECK(seen[b] == 1, "n %d period %d: block %d seen %d times", n, period, b, seen[b]);
        }
    }
    // per-CU stages under the dispatcher model, as cu_balance_period applies
    // it: bh heads a multiple of 8 dividing 256, period 256 / bh, blocks a
    // multiple of the period; block q's stages q + 1 (causal, heaviest first)
    for (int bh : {8, 16, 32, 64, 128}) {
        const int period = 256 / bh;
        for (int nqb = 2 * period; nqb <= 8 * period; nqb += period) {
            std::vector<long long> cu(256, 0);
            for (int y = 0; y < nqb; ++y) {
                for (int h = 0; h < bh; ++h) {
                    const int i = y * bh + h;            // linear work-group index
                    const int xcd = i % 8, slot = (i / 8) % 32;  // dispatch model
                    const int q = nqb - 1 - cu_order_block(y, period);
                    cu[xcd * 32 + slot] += q + 1;
                }
            }
            long long lo = cu[0], hi = cu[0];
            for (int c = 1; c < 256; ++c) {
                lo = cu[c] < lo ? cu[c] : lo;
                hi = cu[c] > hi ? cu[c] : hi;
            }
            const int runs = nqb / period;
            const long long bound = runs % 2 == 0 ? 0 : period - 1;
            CHECK(hi - lo <= bound, "bh %d nqb %d: stages per CU from %lld to %lld (bound %lld)", bh, nqb, lo, hi,
                  bound);
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
