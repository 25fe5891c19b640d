// Buckets of references for the gather form of a scatter (the input
// gradients of the soft backward): given keys[r] in [0, nkeys) for r < R,
// build start[0..nkeys] (exclusive prefix of the bucket sizes) and sorted[]
// where sorted[start[k] .. start[k+1]) lists the r with key k in ascending
// order. The order is fixed, so sums over a bucket are the same on every call.
#pragma once

#include "slg_common.h"

namespace slg {

struct RefTable {
  int* start;   // [nkeys + 1]
  int* sorted;  // [R]
};

// Workspace ints for R references over nkeys buckets (16-byte multiples).
int64_t ref_table_ints(int64_t R, int64_t nkeys);

// Enqueue the build on st; R < 2^31, nkeys < 2^31. Returns 0 or an error.
int build_ref_table(const int* keys, int64_t R, int64_t nkeys, int* ws, hipStream_t st,
                    RefTable* out);

}  // namespace slg
