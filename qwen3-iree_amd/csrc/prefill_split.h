// Key-range splits of the batched prompt attention, shared by the kernel
// (prefill_kernels.hip, where constexpr functions are callable on the device)
// and its launcher (q8gemv_shim.cpp).
//
// Query block q holds tokens 32 q .. 32 q + 31 of the n prompt tokens, at
// positions start + token, and attends cache positions [lo, start + its last
// token] (lo = start or 0).  Counted in blocks of 32 positions from lo that is
//   nb(q) = q + c,  c = 1 + (d + 31) / 32,  d = start - lo,   for q < nqb - 1,
//   nb(nqb - 1) = (d + n - 1) / 32 + 1                      (the last block),
// nqb = ceil(n / 32).  With S blocks per split, query block q has ceil(nb(q) /
// S) splits; the launch enumerates the (query block, split) pairs in order,
// pair p being workgroups (p, kv head) of the grid.
#ifndef QWEN3_PREFILL_SPLIT_H
#define QWEN3_PREFILL_SPLIT_H

#include <stdint.h>

// One split's partial result (f32): O [64 rows][128], m [64], l [64]; rows
// 16 wave + r of the workgroup's four waves.
constexpr int kPfAttnSlotFloats = 64 * 128 + 2 * 64;

// Most K ranges a split attn_o / ffn_down product may have where its reduce
// also forms the following rms_norm (pf_res_reduce_norm keeps every range's
// sums in registers): K <= 3072 gives at most 12 stages of 256.
constexpr int kPfMaxSplits = 12;

struct PfSplitGeometry {
  int32_t nqb;      // query blocks
  int32_t c;        // nb(q) = q + c for q < nqb - 1
  int32_t nb_last;  // nb(nqb - 1)
};

struct PfSplitPair {
  int32_t qb;  // query block
  int32_t s;   // split of it
  int32_t ns;  // its number of splits
};

// n >= 1 tokens at positions start.., 0 <= lo <= start.
constexpr PfSplitGeometry pf_split_geometry(int32_t n, int32_t start, int32_t lo) {
  return PfSplitGeometry{(n + 31) / 32, 1 + (start - lo + 31) / 32, (start - lo + n - 1) / 32 + 1};
}

// sum_{j=1..N} ceil(j / S) for 0 <= N < 2^31, S >= 1
constexpr int64_t pf_ceil_sum(int32_t N, int32_t S) {
  if (N <= 0) return 0;
  const uint32_t a = (uint32_t)N / (uint32_t)S;
  const uint32_t r = (uint32_t)N - a * (uint32_t)S;
  return (int64_t)a * (a + 1) / 2 * S + (int64_t)r * (a + 1);
}

// pairs of query blocks 0 .. q - 1, for q <= nqb - 1
constexpr int64_t pf_pairs_before(const PfSplitGeometry& G, int32_t q, int32_t S) {
  return pf_ceil_sum(G.c + q - 1, S) - pf_ceil_sum(G.c - 1, S);
}

constexpr int64_t pf_pairs_total(const PfSplitGeometry& G, int32_t S) {
  return pf_pairs_before(G, G.nqb - 1, S) + (G.nb_last + S - 1) / S;
}

// the pair with index p (0 <= p < pf_pairs_total)
constexpr PfSplitPair pf_split_pair(const PfSplitGeometry& G, int32_t S, int64_t p) {
  const int64_t before_last = pf_pairs_before(G, G.nqb - 1, S);
  if (p >= before_last)
    return PfSplitPair{G.nqb - 1, (int32_t)(p - before_last), (G.nb_last + S - 1) / S};
  // largest a with pairs_before(a) <= p; pairs_before(nqb - 1) > p
  int32_t a = 0, b = G.nqb - 1;
  while (b - a > 1) {
    const int32_t m = (a + b) / 2;
    if (pf_pairs_before(G, m, S) <= p)
      a = m;
    else
      b = m;
  }
  return PfSplitPair{a, (int32_t)(p - pf_pairs_before(G, a, S)), (a + G.c + S - 1) / S};
}

#endif
