// Bucket table of references (see ref_table.h): counts by key, an exclusive
// scan, placement through atomic cursors, then each bucket put in ascending
// order (placement order varies between calls; the final order does not).
#include "ref_table.h"

namespace slg {

__global__ void __launch_bounds__(256) ref_zero_kernel(int* __restrict__ p, int n) {
  const int t = blockIdx.x * blockDim.x + threadIdx.x;
  if (t < n) p[t] = 0;
}

__global__ void __launch_bounds__(256) ref_count_kernel(const int* __restrict__ keys, int R,
                                                        int* __restrict__ cnt) {
  const int r = blockIdx.x * blockDim.x + threadIdx.x;
  if (r < R) atomicAdd(&cnt[keys[r]], 1);
}

// One workgroup: start[0..n] = exclusive scan of cnt, cursor = start. cnt
// and cursor may be the same array: each element is read before it is
// written, by the one thread that owns it.
__global__ void __launch_bounds__(1024) ref_scan_kernel(const int* cnt, int n,
                                                        int* __restrict__ start, int* cursor) {
  __shared__ int part[1024];
  const int t = threadIdx.x;
  const int per = (n + 1023) / 1024;
  const int lo = min(t * per, n), hi = min(lo + per, n);
  int sum = 0;
  for (int i = lo; i < hi; ++i) sum += cnt[i];
  part[t] = sum;
  __syncthreads();
  for (int d = 1; d < 1024; d <<= 1) {  // inclusive Hillis-Steele scan
    const int v = t >= d ? part[t - d] : 0;
    __syncthreads();
    part[t] += v;
    __syncthreads();
  }
  int run = part[t] - sum;
  for (int i = lo; i < hi; ++i) {
    const int c = cnt[i];
    start[i] = run;
    cursor[i] = run;
    run += c;
  }
  if (t == 1023) start[n] = part[1023];
}

__global__ void __launch_bounds__(256) ref_fill_kernel(const int* __restrict__ keys, int R,
                                                       int* __restrict__ cursor,
                                                       int* __restrict__ refs) {
  const int r = blockIdx.x * blockDim.x + threadIdx.x;
  if (r < R) refs[atomicAdd(&cursor[keys[r]], 1)] = r;
}

__device__ inline void sift_down(int* a, int root, int n) {
  const int v = a[root];
  for (;;) {
    int c = 2 * root + 1;
    if (c >= n) break;
    if (c + 1 < n && a[c + 1] > a[c]) ++c;
    if (a[c] <= v) break;
    a[root] = a[c];
    root = c;
  }
  a[root] = v;
}

// One wave per bucket. Buckets of up to kRankCap references are copied to
// LDS and each element goes to its rank (the count of smaller references;
// references are distinct), so the wave's reads are independent broadcasts;
// larger buckets are heap-sorted in place by one lane.
constexpr int kRankCap = 512;

__global__ void __launch_bounds__(256) ref_rank_kernel(const int* __restrict__ start, int n_keys,
                                                       int* __restrict__ refs,
                                                       int* __restrict__ sorted) {
  __shared__ int buf[4][kRankCap];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int k = blockIdx.x * 4 + wave;
  const int s = k < n_keys ? start[k] : 0;
  const int n = k < n_keys ? start[k + 1] - s : 0;
  int* a = refs + s;
  int* bw = buf[wave];
  const bool small = n <= kRankCap;
  if (small) {
    for (int j = lane; j < n; j += 64) bw[j] = a[j];
  } else if (lane == 0) {
    for (int r = n / 2 - 1; r >= 0; --r) sift_down(a, r, n);
    for (int e = n - 1; e > 0; --e) {
      const int t = a[0];
      a[0] = a[e];
      a[e] = t;
      sift_down(a, 0, e);
    }
  }
  __syncthreads();  // LDS copies and the in-place sorts are visible to the workgroup
  for (int j = lane; j < n; j += 64) {
    if (small) {
      const int r = bw[j];
      int pos = 0;
      for (int t = 0; t < n; ++t) pos += bw[t] < r;
      sorted[s + pos] = r;
    } else {
      sorted[s + j] = a[j];
    }
  }
}

static inline int64_t round4i(int64_t n) { return (n + 3) & ~int64_t(3); }

int64_t ref_table_ints(int64_t R, int64_t nkeys) {
  return round4i(nkeys + 1) + round4i(nkeys) + 2 * round4i(R);
}

int build_ref_table(const int* keys, int64_t R, int64_t nkeys, int* ws, hipStream_t st,
                    RefTable* out) {
  SLG_REQUIRE(R >= 0 && R < (1LL << 31) && nkeys > 0 && nkeys < (1LL << 31), SLG_E_SHAPE,
              "reference table: %lld references over %lld keys", (long long)R,
              (long long)nkeys);
  int* start = ws;
  int* cursor = start + round4i(nkeys + 1);
  int* refs = cursor + round4i(nkeys);
  int* sorted = refs + round4i(R);
  hipLaunchKernelGGL(ref_zero_kernel, dim3((unsigned)cdiv(nkeys, 256)), dim3(256), 0, st, cursor,
                     (int)nkeys);
  if (R > 0)
    hipLaunchKernelGGL(ref_count_kernel, dim3((unsigned)cdiv(R, 256)), dim3(256), 0, st, keys,
                       (int)R, cursor);
  hipLaunchKernelGGL(ref_scan_kernel, dim3(1), dim3(1024), 0, st, cursor, (int)nkeys, start,
                     cursor);
  if (R > 0) {
    hipLaunchKernelGGL(ref_fill_kernel, dim3((unsigned)cdiv(R, 256)), dim3(256), 0, st, keys,
                       (int)R, cursor, refs);
    hipLaunchKernelGGL(ref_rank_kernel, dim3((unsigned)cdiv(nkeys, 4)), dim3(256), 0, st, start,
                       (int)nkeys, refs, sorted);
  }
  SLG_LAUNCH_CHECK("reference table");
  out->start = start;
  out->sorted = sorted;
  return 0;
}

}  // namespace slg
