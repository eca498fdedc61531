// Brute-force check of prefill_split.h: for many prompt shapes and split
// sizes, the closed-form pair count and the pair -> (query block, split)
// mapping against a direct enumeration of the query blocks' position ranges.
#include <cstdio>
#include <vector>

#include "prefill_split.h"

static int check(int n, int start, int lo, int S) {
  const PfSplitGeometry G = pf_split_geometry(n, start, lo);
  std::vector<PfSplitPair> want;
  const int nqb = (n + 31) / 32;
  for (int q = 0; q < nqb; ++q) {
    const int last_tok = 32 * q + 31 < n ? 32 * q + 31 : n - 1;
    const int hi = start + last_tok;
    int nb = 0;  // blocks of 32 positions from lo that [lo, hi] touches
    for (int p = lo; p <= hi; p += 32) ++nb;
    const int ns = (nb + S - 1) / S;
    for (int s = 0; s < ns; ++s) want.push_back(PfSplitPair{q, s, ns});
  }
  if (G.nqb != nqb || pf_pairs_total(G, S) != (int64_t)want.size()) {
    std::printf("total n=%d start=%d lo=%d S=%d: %lld != %zu\n", n, start, lo, S,
                (long long)pf_pairs_total(G, S), want.size());
    return 1;
  }
  for (size_t p = 0; p < want.size(); ++p) {
    const PfSplitPair got = pf_split_pair(G, S, (int64_t)p);
    if (got.qb != want[p].qb || got.s != want[p].s || got.ns != want[p].ns) {
      std::printf("pair %zu n=%d start=%d lo=%d S=%d: (%d %d %d) != (%d %d %d)\n", p, n, start,
                  lo, S, got.qb, got.s, got.ns, want[p].qb, want[p].s, want[p].ns);
      return 1;
    }
  }
  return 0;
}

int main() {
  long cases = 0;
  const int ns[] = {1, 2, 31, 32, 33, 63, 64, 65, 100, 512, 777, 2048};
  const int starts[] = {0, 1, 5, 31, 32, 33, 100, 1000};
  const int splits[] = {1, 2, 3, 4, 7, 16, 64, 1000};
  for (int n : ns)
    for (int start : starts)
      for (int local = 0; local < 2; ++local)
        for (int S : splits) {
          if (check(n, start, local ? start : 0, S)) return 1;
          ++cases;
        }
  // the sum formula against direct sums
  for (int S = 1; S < 40; ++S)
    for (int N = 0; N < 300; ++N) {
      int64_t direct = 0;
      for (int j = 1; j <= N; ++j) direct += (j + S - 1) / S;
      if (pf_ceil_sum(N, S) != direct) {
        std::printf("ceil_sum N=%d S=%d\n", N, S);
        return 1;
      }
    }
  std::printf("ok %ld cases\n", cases);
  return 0;
}
