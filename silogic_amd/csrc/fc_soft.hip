// FC soft forward for gfx950: Top-K gather + 4-coefficient node, and the
// parameter prep / GroupSum kernels around it.
//
// Design (one layer, x [B,IN] -> y [B,OUT]):
//   * A workgroup owns a tile of S consecutive samples and a chunk of
//     outputs. It stages the S input rows in LDS transposed, group-major:
//     lds[g][i] = the V = min(S,4) samples 4g..4g+V-1 of input i, so one
//     ds_read_b128 per candidate fetches 4 samples. Random-address b128
//     reads are the widest LDS gather gfx950 has; b64 and b32 move fewer
//     bytes per LDS cycle.
//   * Lanes walk outputs. Each lane loads its output's 2K candidate indices,
//     2K weights and 4 node coefficients with 16-byte loads and reuses them
//     for all S samples: 144 B at K = 8 from the separate arrays, 112
//     contiguous bytes from a per-output record (slg_fc_soft_records, the
//     indices as 16-bit pairs).
//   * Output stores are coalesced along the output dimension. The fused
//     GroupSum variant stores nothing per output: it counts (y > 0.5) per
//     class with a wave ballot + popcount into LDS counters and writes the
//     [S, C] logits of its tile at the end.
//   * The tile/chunk index is remapped so chunks of one tile run on the same
//     XCD and share its L2 copy of the input rows.
#include "fc_soft_common.h"

namespace slg {

// Fused GroupSum head (heads.py:34-39 with the feature STE): per-class
// counts of (y > 0.5), logits = count / tau.
struct HeadArgs {
  float* logits;
  int C;
  int per;  // OUT / C outputs per class
  float tau;
};

// Widest workgroup per variant: 1024 threads keeps <= 128 VGPRs per lane,
// which fits the lean variants; the others get 512 threads and more registers.
template <int KC, int S>
constexpr int soft_max_threads() { return (KC == 0 || S >= 8) ? 512 : 1024; }

template <int NODE, int KC, int S, bool HEAD, bool REC>
__global__ void __launch_bounds__((soft_max_threads<KC, S>()))
fc_soft_kernel(const float* __restrict__ x, int B, int IN, int OUT, int Kr, ParamView pv,
               float inv_tau, float* __restrict__ y, int n_chunks, int chunk, HeadArgs hd) {
  constexpr int V = S >= 4 ? 4 : S;
  constexpr int G = S / V;
  constexpr int KM = KC > 0 ? KC : 16;
  using vt = typename vecf<V>::t;
  extern __shared__ __align__(16) unsigned char smem[];
  vt* lds = reinterpret_cast<vt*>(smem);
  unsigned* cnt = reinterpret_cast<unsigned*>(smem + (size_t)IN * S * sizeof(float));
  const int K = KC > 0 ? KC : Kr;

  const uint32_t lid = xcd_logical_id(blockIdx.x, gridDim.x);
  const int tile = (int)(lid / (uint32_t)n_chunks);
  const int ch = (int)(lid % (uint32_t)n_chunks);
  const int b0 = tile * S;
  const int o_begin = ch * chunk;
  const int o_end = min(OUT, o_begin + chunk);

  if constexpr (HEAD) {
    for (int t = threadIdx.x; t < S * hd.C; t += blockDim.x) cnt[t] = 0u;
  }

  // Stage S rows transposed: lds[g * IN + i] holds samples b0+gV .. b0+gV+V-1
  // of input i.
  for (int g = 0; g < G; ++g) stage_rows<V, true>(lds + g * IN, x, B, IN, b0 + g * V);
  __syncthreads();

  const uint32_t lim = (uint32_t)IN - 1u;
  const int lane = threadIdx.x & 63;
  // The tile's output rows as a buffer resource (S * OUT * 4 < 2^31 bytes,
  // checked at launch): stores past its valid rows are dropped.
  __amdgpu_buffer_rsrc_t yrows;
  if constexpr (!HEAD)
    yrows = uniform_rsrc(y + (int64_t)min(b0, B) * OUT, max(0, min(S, B - b0)) * OUT * 4);

  // Each wave owns a contiguous run of 64-output chunks; lane = output
  // within a chunk. The next chunk's parameters are loaded while this one
  // computes (two register sets, no copies); loads past the end re-read the
  // last output, so every load is in bounds and unconditional.
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  const int nwaves = blockDim.x >> 6;
  const int n64 = (o_end - o_begin + 63) >> 6;
  const int cpw = (n64 + nwaves - 1) / nwaves;
  const int j_begin = wave * cpw, j_end = min(n64, j_begin + cpw);
  const int o_last = o_end - 1;

  // Fused head: per-sample counts of the current class in scalar registers,
  // added to the LDS counters when the chunk run leaves the class. A chunk
  // that straddles a class boundary counts lane by lane with LDS atomics.
  int cur_c = 0, hi_b = 0;
  unsigned acc[S];
#pragma unroll
  for (int s = 0; s < S; ++s) acc[s] = 0u;
  if constexpr (HEAD) {
    if (j_begin < j_end) {
      cur_c = (o_begin + j_begin * 64) / hd.per;
      hi_b = (cur_c + 1) * hd.per;
    }
  }

  auto chunk_body = [&](const FcParams<KM>& P, int jj) {
    const int oc0 = o_begin + jj * 64;
    const int o = oc0 + lane;
    const bool valid = o < o_end;
    // clamp into the staged rows (unsigned min also maps negatives to IN-1)
    // (records hold indices the records kernel already clamped)
    uint32_t ia[KM], ib[KM];
#pragma unroll
    for (int k = 0; k < KM; ++k) {
      ia[k] = REC ? (uint32_t)P.ia[k] : min((uint32_t)P.ia[k], lim);
      ib[k] = REC ? (uint32_t)P.ib[k] : min((uint32_t)P.ib[k], lim);
    }
    float yv[S];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const vt* src = lds + g * IN;
      // slot a, then slot b: at most K gathers in flight per wave keeps the
      // two parameter sets and the gathered vectors within 128 VGPRs
      vt A = zero_vec<vt>(), Bv = zero_vec<vt>();
#pragma unroll
      for (int k = 0; k < KM; ++k)
        if (KC > 0 || k < K) fma_acc(A, P.fa[k], src[ia[k]]);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int k = 0; k < KM; ++k)
        if (KC > 0 || k < K) fma_acc(Bv, P.fb[k], src[ib[k]]);
#pragma unroll
      for (int v = 0; v < V; ++v)
        yv[g * V + v] = node_eval<NODE>(lanev(A, v), lanev(Bv, v), P.p, inv_tau);
    }
    if constexpr (HEAD) {
      const int oc1 = min(oc0 + 63, o_last);
      if (oc1 < hi_b) {  // the whole chunk lies in class cur_c (wave-uniform)
#pragma unroll
        for (int s = 0; s < S; ++s)
          acc[s] += (unsigned)__popcll(__ballot(valid && b0 + s < B && yv[s] > 0.5f));
      } else {
        if (lane == 0) {
#pragma unroll
          for (int s = 0; s < S; ++s)
            if (acc[s]) atomicAdd(&cnt[s * hd.C + cur_c], acc[s]);
        }
#pragma unroll
        for (int s = 0; s < S; ++s) acc[s] = 0u;
        if (valid) {
          const int c = o / hd.per;
#pragma unroll
          for (int s = 0; s < S; ++s)
            if (b0 + s < B && yv[s] > 0.5f) atomicAdd(&cnt[s * hd.C + c], 1u);
        }
        cur_c = (oc1 + 1) / hd.per;  // class of the wave's next output
        hi_b = (cur_c + 1) * hd.per;
      }
    } else {
      // branch-free stores: lanes past the chunk and rows past the batch
      // fall outside the tile's resource and are dropped by the hardware
      const uint32_t vo = valid ? (uint32_t)o * 4u : 0x80000000u;
#pragma unroll
      for (int s = 0; s < S; ++s)
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(yv[s]), yrows,
                                              (int)(vo + (uint32_t)(s * OUT) * 4u), 0, 0);
    }
  };

  if (j_begin < j_end) {
    FcParams<KM> P, Q;
    int jj = j_begin;
    load_params<KC, KM, REC>(P, min(o_begin + jj * 64 + lane, o_last), K, pv);
    while (true) {
      load_params<KC, KM, REC>(Q, min(o_begin + (jj + 1) * 64 + lane, o_last), K, pv);
      chunk_body(P, jj);
      if (++jj >= j_end) break;
      load_params<KC, KM, REC>(P, min(o_begin + (jj + 1) * 64 + lane, o_last), K, pv);
      chunk_body(Q, jj);
      if (++jj >= j_end) break;
    }
    if constexpr (HEAD) {
      if (lane == 0) {
#pragma unroll
        for (int s = 0; s < S; ++s)
          if (acc[s]) atomicAdd(&cnt[s * hd.C + cur_c], acc[s]);
      }
    }
  }
  if constexpr (HEAD) {
    __syncthreads();
    for (int t = threadIdx.x; t < S * hd.C; t += blockDim.x) {
      const int s = t / hd.C, c = t % hd.C;
      if (b0 + s < B) hd.logits[(int64_t)(b0 + s) * hd.C + c] = (float)cnt[t] / hd.tau;
    }
  }
}

// Index half of a record word, pre-scaled to a byte offset into the staged
// tile (slot = 4V bytes): one SDWA shift reads the 16-bit half in place.
template <int SH>
__device__ inline uint32_t idx_lo_bytes(uint32_t w) {
  uint32_t r;
  asm("v_lshlrev_b32_sdwa %0, %1, %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD "
      "src1_sel:WORD_0"
      : "=v"(r) : "i"(SH), "v"(w));
  return r;
}
template <int SH>
__device__ inline uint32_t idx_hi_bytes(uint32_t w) {
  uint32_t r;
  asm("v_lshlrev_b32_sdwa %0, %1, %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD "
      "src1_sel:WORD_1"
      : "=v"(r) : "i"(SH), "v"(w));
  return r;
}

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

// LDS read at a byte offset from the start of the workgroup's LDS. The
// records kernel declares no static LDS, so its dynamic tile starts at LDS
// address 0 (checked at launch) and the offset is the address itself.
template <typename T>
__device__ inline T lds_at(uint32_t off) {
  return *reinterpret_cast<const __attribute__((address_space(3))) T*>((uintptr_t)off);
}

// Soft forward over records with KC = 4 or 8 candidates per slot: the
// arithmetic of fc_soft_kernel<.., REC> (the same fmaf sequence per output
// and sample, so bit-identical results) with fewer VALU and memory
// instructions per 64-output chunk:
//  * a chunk's record quads are read through a buffer resource at a
//    wave-uniform offset (chunk * quads * 1 KB) plus the lane's 16 bytes, so
//    no per-lane address arithmetic; the next chunk's quads load while this
//    one computes, the first chunk's during staging;
//  * index halves become LDS byte offsets with one SDWA shift each;
//  * a slot's KC gathers are issued together before they are accumulated;
//  * stores take the sample row as a scalar offset.
template <int NODE, int KC, int S, bool HEAD>
__global__ void __launch_bounds__((soft_max_threads<KC, S>()))
fc_soft_rec_kernel(const float* __restrict__ x, int B, int IN, int OUT,
                   const uint32_t* __restrict__ rec, float inv_tau, float* __restrict__ y,
                   int n_chunks, int chunk, HeadArgs hd) {
  static_assert(KC == 4 || KC == 8, "records kernel takes 4 or 8 candidates");
  constexpr int V = S >= 4 ? 4 : S;
  constexpr int G = S / V;
  constexpr int RQ = rec_quads(KC);
  constexpr int SH = V == 4 ? 4 : (V == 2 ? 3 : 2);  // log2 of the slot bytes
  using vt = typename vecf<V>::t;
  extern __shared__ __align__(16) unsigned char smem[];
  vt* lds = reinterpret_cast<vt*>(smem);
  unsigned* cnt = reinterpret_cast<unsigned*>(smem + (size_t)IN * S * sizeof(float));

  const uint32_t lid = xcd_logical_id(blockIdx.x, gridDim.x);
  const int tile = (int)(lid / (uint32_t)n_chunks);
  const int ch = (int)(lid % (uint32_t)n_chunks);
  const int b0 = tile * S;
  const int rows = min(S, B - b0);  // valid rows of the tile (>= 1)
  const int o_begin = ch * chunk;   // a multiple of 64
  const int o_end = min(OUT, o_begin + chunk);
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nwaves = blockDim.x >> 6;
  const int n64 = (o_end - o_begin + 63) >> 6;
  const int cpw = (n64 + nwaves - 1) / nwaves;
  const int j_begin = wave * cpw, j_end = min(n64, j_begin + cpw);
  const int c0 = o_begin >> 6;                // layer chunk of jj = 0
  const int c_last = ((OUT + 63) >> 6) - 1;   // last chunk with records

  if constexpr (HEAD) {
    for (int t = threadIdx.x; t < S * hd.C; t += blockDim.x) cnt[t] = 0u;
  }

  const __amdgpu_buffer_rsrc_t rr = uniform_rsrc(rec, (c_last + 1) * RQ * 1024);
  const int lane16 = lane * 16;
  auto load_rec = [&](u32x4 (&R)[RQ], int c) {  // c wave-uniform
    const int so = min(c, c_last) * (RQ * 1024);
#pragma unroll
    for (int q = 0; q < RQ; ++q)
      R[q] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rr, lane16, so + q * 1024, 0));
  };
  u32x4 P[RQ], Q[RQ];
  if (j_begin < j_end) load_rec(P, c0 + j_begin);

  // every staging load of the tile in flight at once (one pass of NB
  // batches covers the widest rows of each tile size at 1024 threads)
  constexpr int NB = V == 4 ? 3 : (V == 2 ? 5 : 10);
  for (int g = 0; g < G; ++g) stage_rows<V, true, NB>(lds + g * IN, x, B, IN, b0 + g * V);
  __syncthreads();

  __amdgpu_buffer_rsrc_t yrows;
  if constexpr (!HEAD) yrows = uniform_rsrc(y + (int64_t)b0 * OUT, rows * OUT * 4);

  int cur_c = 0, hi_b = 0;
  unsigned acc[S];
#pragma unroll
  for (int s = 0; s < S; ++s) acc[s] = 0u;
  if constexpr (HEAD) {
    if (j_begin < j_end) {
      cur_c = (o_begin + j_begin * 64) / hd.per;
      hi_b = (cur_c + 1) * hd.per;
    }
  }
  const uint32_t gstride = (uint32_t)IN * (uint32_t)sizeof(vt);

  auto chunk_body = [&](const u32x4 (&R)[RQ], int jj) {
    const int oc0 = o_begin + jj * 64;
    const int o = oc0 + lane;
    const bool valid = o < o_end;
    auto word = [&](int w) { return R[w >> 2][w & 3]; };
    float yv[S];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      vt A = zero_vec<vt>(), Bv = zero_vec<vt>();
      {
        vt ga[KC];
#pragma unroll
        for (int k = 0; k < KC; ++k) ga[k] = lds_at<vt>(idx_lo_bytes<SH>(word(k)) + g * gstride);
#pragma unroll
        for (int k = 0; k < KC; ++k) fma_acc(A, __uint_as_float(word(KC + k)), ga[k]);
      }
      // slot a is accumulated before slot b's gathers go out, which reuse
      // its registers (KC reads in flight, no spills at 128 VGPRs)
      asm volatile("" : "+v"(A)::"memory");
      {
        vt gb[KC];
#pragma unroll
        for (int k = 0; k < KC; ++k) gb[k] = lds_at<vt>(idx_hi_bytes<SH>(word(k)) + g * gstride);
#pragma unroll
        for (int k = 0; k < KC; ++k) fma_acc(Bv, __uint_as_float(word(2 * KC + k)), gb[k]);
      }
      const float4 p = make_float4(__uint_as_float(word(4 * (RQ - 1))),
                                   __uint_as_float(word(4 * (RQ - 1) + 1)),
                                   __uint_as_float(word(4 * (RQ - 1) + 2)),
                                   __uint_as_float(word(4 * (RQ - 1) + 3)));
#pragma unroll
      for (int v = 0; v < V; ++v)
        yv[g * V + v] = node_eval<NODE>(lanev(A, v), lanev(Bv, v), p, inv_tau);
    }
    if constexpr (HEAD) {
      const int oc1 = min(oc0 + 63, o_end - 1);
      if (oc1 < hi_b) {  // the whole chunk lies in class cur_c (wave-uniform)
#pragma unroll
        for (int s = 0; s < S; ++s)
          acc[s] += (unsigned)__popcll(__ballot(valid && s < rows && yv[s] > 0.5f));
      } else {
        if (lane == 0) {
#pragma unroll
          for (int s = 0; s < S; ++s)
            if (acc[s]) atomicAdd(&cnt[s * hd.C + cur_c], acc[s]);
        }
#pragma unroll
        for (int s = 0; s < S; ++s) acc[s] = 0u;
        if (valid) {
          const int c = o / hd.per;
#pragma unroll
          for (int s = 0; s < S; ++s)
            if (s < rows && yv[s] > 0.5f) atomicAdd(&cnt[s * hd.C + c], 1u);
        }
        cur_c = (oc1 + 1) / hd.per;  // class of the wave's next output
        hi_b = (cur_c + 1) * hd.per;
      }
    } else {
      // lanes past the chunk fall outside the resource and are dropped;
      // rows past the batch are skipped (wave-uniform)
      const uint32_t vo = valid ? (uint32_t)o * 4u : 0x80000000u;
#pragma unroll
      for (int s = 0; s < S; ++s)
        if (s < rows)
          __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(yv[s]), yrows, (int)vo,
                                                s * OUT * 4, 0);
    }
  };

  if (j_begin < j_end) {
    int jj = j_begin;
    while (true) {
      load_rec(Q, c0 + jj + 1);
      chunk_body(P, jj);
      if (++jj >= j_end) break;
      load_rec(P, c0 + jj + 1);
      chunk_body(Q, jj);
      if (++jj >= j_end) break;
    }
    if constexpr (HEAD) {
      if (lane == 0) {
#pragma unroll
        for (int s = 0; s < S; ++s)
          if (acc[s]) atomicAdd(&cnt[s * hd.C + cur_c], acc[s]);
      }
    }
  }
  if constexpr (HEAD) {
    __syncthreads();
    for (int t = threadIdx.x; t < S * hd.C; t += blockDim.x) {
      const int s = t / hd.C, c = t % hd.C;
      if (b0 + s < B) hd.logits[(int64_t)(b0 + s) * hd.C + c] = (float)cnt[t] / hd.tau;
    }
  }
}

// ---------------------------------------------------------------------------
// A whole narrow network in one launch (small batches)
// ---------------------------------------------------------------------------
// With few samples a launch per layer is mostly latency: staging, record
// loads and the launch itself. Here a workgroup takes 4 samples through
// every layer: the activations stay in LDS (two buffers of float4 slots, one
// per input, ping-ponged), each layer reads its records as the records
// kernel does and accumulates in the same order (the same bits per layer),
// and the last layer either writes its activations or, with the STE GroupSum
// head, only the per-class counts (wave ballots into LDS counters, integers,
// so exact) / tau.
constexpr int kMaxNetLayers = 16;
constexpr int kNetSoftThreads = 1024;
struct SoftNetDesc {
  const float* rec[kMaxNetLayers];
  int out_dim[kMaxNetLayers];
  int L, K, maxw;   // maxw: float4 slots per activation buffer
  float inv_tau;
};

template <int NODE, int KC, bool HEAD>
__global__ void __launch_bounds__(kNetSoftThreads)
fc_soft_net_kernel(const float* __restrict__ x, int B, int IN, SoftNetDesc d,
                   float* __restrict__ y, HeadArgs hd) {
  constexpr int KM = KC > 0 ? KC : 16;
  extern __shared__ __align__(16) unsigned char smem[];
  f32x4* cur = reinterpret_cast<f32x4*>(smem);
  f32x4* nxt = cur + d.maxw;
  unsigned* cnt = reinterpret_cast<unsigned*>(cur + 2 * d.maxw);
  const int K = KC > 0 ? KC : d.K;
  const int b0 = blockIdx.x * 4;
  const int lane = threadIdx.x & 63;
  if constexpr (HEAD) {
    for (int t = threadIdx.x; t < 4 * hd.C; t += blockDim.x) cnt[t] = 0u;
  }
  stage_rows<4, true>(cur, x, B, IN, b0);
  __syncthreads();
  for (int l = 0; l < d.L; ++l) {
    const int OUT = d.out_dim[l];
    const bool last = l + 1 == d.L;
    ParamView pv{};
    pv.rec = d.rec[l];
    // whole waves iterate (the head's ballots need every lane)
    const int n_iter = (OUT + (int)blockDim.x - 1) / (int)blockDim.x;
    for (int it = 0; it < n_iter; ++it) {
      const int o = it * (int)blockDim.x + (int)threadIdx.x;
      const bool valid = o < OUT;
      FcParams<KM> P;
      load_params<KC, KM, true>(P, min(o, OUT - 1), K, pv);
      f32x4 A = zero_vec<f32x4>(), Bv = zero_vec<f32x4>();
#pragma unroll
      for (int k = 0; k < KM; ++k)
        if (KC > 0 || k < K) fma_acc(A, P.fa[k], cur[P.ia[k]]);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int k = 0; k < KM; ++k)
        if (KC > 0 || k < K) fma_acc(Bv, P.fb[k], cur[P.ib[k]]);
      float yv[4];
#pragma unroll
      for (int v = 0; v < 4; ++v) yv[v] = node_eval<NODE>(A[v], Bv[v], P.p, d.inv_tau);
      if (!last) {
        if (valid) nxt[o] = f32x4{yv[0], yv[1], yv[2], yv[3]};
      } else if constexpr (HEAD) {
        const int c = valid ? o / hd.per : -1;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const bool hit = valid && b0 + s < B && yv[s] > 0.5f;
          uint64_t todo = __ballot(valid);
          while (todo) {   // the classes this wave's outputs fall in, in order
            const int cc = __shfl(c, __ffsll((long long)todo) - 1);
            const uint64_t mine = __ballot(c == cc);
            const unsigned n = (unsigned)__popcll(__ballot(hit && c == cc));
            if (lane == 0 && n) atomicAdd(&cnt[s * hd.C + cc], n);
            todo &= ~mine;
          }
        }
      } else {
        if (valid) {
#pragma unroll
          for (int s = 0; s < 4; ++s)
            if (b0 + s < B) y[(int64_t)(b0 + s) * OUT + o] = yv[s];
        }
      }
    }
    __syncthreads();
    f32x4* t = cur;
    cur = nxt;
    nxt = t;
  }
  if constexpr (HEAD) {
    for (int t = threadIdx.x; t < 4 * hd.C; t += blockDim.x) {
      const int s = t / hd.C, c = t % hd.C;
      if (b0 + s < B) hd.logits[(int64_t)(b0 + s) * hd.C + c] = (float)cnt[t] / hd.tau;
    }
  }
}

// ---------------------------------------------------------------------------
// A whole wide network per sample tile (large batches)
// ---------------------------------------------------------------------------
// A layer launched on its own stages its S-sample tile from HBM, computes
// every output and writes them back: at config 2 (10000-wide layers, 4-sample
// tiles) the staging cannot overlap the compute (the tile fills LDS) and
// costs about a quarter of the layer. Here a workgroup takes its tile through
// every layer with one LDS buffer: a layer computes all of the tile's
// outputs with fc_soft_rec_kernel's arithmetic (same records, the same fmaf
// sequence per output and sample, so the same bits), holds them in
// registers (each wave its CPW chunks of 64 outputs, S values per lane and
// chunk), and after a barrier writes them over its input. HBM then sees the
// first layer's input rows and the logits (or the last activations) only;
// what remains per layer is the record stream from L2 and the LDS gathers.
constexpr int kRecNetThreads = 512;
struct RecNetDesc {
  const uint32_t* rec[kMaxNetLayers];
  int out_dim[kMaxNetLayers];
  int L;
  float inv_tau;
};

template <int NODE, int KC, int S, int CPW, bool HEAD>
__global__ void __launch_bounds__(kRecNetThreads)
fc_soft_rec_net_kernel(const float* __restrict__ x, int B, int IN, RecNetDesc d,
                       float* __restrict__ y, int maxw, HeadArgs hd) {
  static_assert(KC == 4 || KC == 8, "records take 4 or 8 candidates");
  static_assert(S == 2 || S == 4, "tiles of 2 or 4 samples");
  constexpr int RQ = rec_quads(KC);
  constexpr int SH = S == 4 ? 4 : 3;  // log2 of the slot bytes
  using vt = typename vecf<S>::t;
  extern __shared__ __align__(16) unsigned char smem[];
  vt* lds = reinterpret_cast<vt*>(smem);
  unsigned* cnt = reinterpret_cast<unsigned*>(smem + (size_t)maxw * S * sizeof(float));
  const int b0 = blockIdx.x * S;
  const int rows = min(S, B - b0);
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  constexpr int nwaves = kRecNetThreads / 64;
  const int lane16 = lane * 16;
  if constexpr (HEAD) {
    for (int t = threadIdx.x; t < S * hd.C; t += blockDim.x) cnt[t] = 0u;
  }

  // a chunk's record quads: wave-uniform offset + the lane's 16 bytes
  auto load_rec = [&](u32x4 (&R)[RQ], const __amdgpu_buffer_rsrc_t& rr, int c, int c_last) {
    const int so = min(c, c_last) * (RQ * 1024);
#pragma unroll
    for (int q = 0; q < RQ; ++q)
      R[q] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rr, lane16, so + q * 1024, 0));
  };
  // one chunk of 64 outputs for the tile's S samples (fc_soft_rec_kernel's
  // chunk arithmetic)
  auto chunk_vals = [&](const u32x4 (&R)[RQ], float (&yv)[S]) __attribute__((always_inline)) {
    auto word = [&](int w) { return R[w >> 2][w & 3]; };
    vt A = zero_vec<vt>(), Bv = zero_vec<vt>();
    {
      vt ga[KC];
#pragma unroll
      for (int k = 0; k < KC; ++k) ga[k] = lds_at<vt>(idx_lo_bytes<SH>(word(k)));
#pragma unroll
      for (int k = 0; k < KC; ++k) fma_acc(A, __uint_as_float(word(KC + k)), ga[k]);
    }
    asm volatile("" : "+v"(A)::"memory");
    {
      vt gb[KC];
#pragma unroll
      for (int k = 0; k < KC; ++k) gb[k] = lds_at<vt>(idx_hi_bytes<SH>(word(k)));
#pragma unroll
      for (int k = 0; k < KC; ++k) fma_acc(Bv, __uint_as_float(word(2 * KC + k)), gb[k]);
    }
    const float4 p = make_float4(__uint_as_float(word(4 * (RQ - 1))),
                                 __uint_as_float(word(4 * (RQ - 1) + 1)),
                                 __uint_as_float(word(4 * (RQ - 1) + 2)),
                                 __uint_as_float(word(4 * (RQ - 1) + 3)));
#pragma unroll
    for (int v = 0; v < S; ++v) yv[v] = node_eval<NODE>(lanev(A, v), lanev(Bv, v), p, d.inv_tau);
  };

  constexpr int NB = S == 4 ? 3 : 5;
  stage_rows<S, true, NB>(lds, x, B, IN, b0);
  __syncthreads();

  // every layer but the last: outputs held in registers, then written over
  // the tile after every wave has read it
  for (int l = 0; l + 1 < d.L; ++l) {
    const int OUT = d.out_dim[l];
    const int n64 = (OUT + 63) >> 6;
    const int cpw = (n64 + nwaves - 1) / nwaves;   // <= CPW (checked on the host)
    const int j_begin = wave * cpw, j_end = min(n64, j_begin + cpw);
    const __amdgpu_buffer_rsrc_t rr = uniform_rsrc(d.rec[l], n64 * RQ * 1024);
    u32x4 R[2][RQ];
    float res[CPW][S];
    if (j_begin < j_end) load_rec(R[0], rr, j_begin, n64 - 1);
#pragma unroll
    for (int jj = 0; jj < CPW; ++jj) {
      if (j_begin + jj < j_end) {
        load_rec(R[(jj + 1) & 1], rr, j_begin + jj + 1, n64 - 1);
        chunk_vals(R[jj & 1], res[jj]);
      }
    }
    __syncthreads();
#pragma unroll
    for (int jj = 0; jj < CPW; ++jj) {
      const int o = (j_begin + jj) * 64 + lane;
      if (j_begin + jj < j_end && o < OUT) lds[o] = make_vec<S>(res[jj]);
    }
    __syncthreads();
  }

  // the last layer: the STE GroupSum's class counts, or the activations
  {
    const int l = d.L - 1;
    const int OUT = d.out_dim[l];
    const int n64 = (OUT + 63) >> 6;
    const int cpw = (n64 + nwaves - 1) / nwaves;
    const int j_begin = wave * cpw, j_end = min(n64, j_begin + cpw);
    const __amdgpu_buffer_rsrc_t rr = uniform_rsrc(d.rec[l], n64 * RQ * 1024);
    __amdgpu_buffer_rsrc_t yrows;
    if constexpr (!HEAD) yrows = uniform_rsrc(y + (int64_t)b0 * OUT, rows * OUT * 4);
    int cur_c = 0, hi_b = 0;
    unsigned acc[S];
#pragma unroll
    for (int s = 0; s < S; ++s) acc[s] = 0u;
    if constexpr (HEAD) {
      if (j_begin < j_end) {
        cur_c = (j_begin * 64) / hd.per;
        hi_b = (cur_c + 1) * hd.per;
      }
    }
    u32x4 P[RQ], Q[RQ];
    auto emit = [&](const u32x4 (&R)[RQ], int j) __attribute__((always_inline)) {
      float yv[S];
      chunk_vals(R, yv);
      const int oc0 = j * 64;
      const int o = oc0 + lane;
      const bool valid = o < OUT;
      if constexpr (HEAD) {
        const int oc1 = min(oc0 + 63, OUT - 1);
        if (oc1 < hi_b) {  // the whole chunk lies in class cur_c (wave-uniform)
#pragma unroll
          for (int s = 0; s < S; ++s)
            acc[s] += (unsigned)__popcll(__ballot(valid && s < rows && yv[s] > 0.5f));
        } else {
          if (lane == 0) {
#pragma unroll
            for (int s = 0; s < S; ++s)
              if (acc[s]) atomicAdd(&cnt[s * hd.C + cur_c], acc[s]);
          }
#pragma unroll
          for (int s = 0; s < S; ++s) acc[s] = 0u;
          if (valid) {
            const int c = o / hd.per;
#pragma unroll
            for (int s = 0; s < S; ++s)
              if (s < rows && yv[s] > 0.5f) atomicAdd(&cnt[s * hd.C + c], 1u);
          }
          cur_c = (oc1 + 1) / hd.per;
          hi_b = (cur_c + 1) * hd.per;
        }
      } else {
        const uint32_t vo = valid ? (uint32_t)o * 4u : 0x80000000u;
#pragma unroll
        for (int s = 0; s < S; ++s)
          if (s < rows)
            __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(yv[s]), yrows, (int)vo,
                                                  s * OUT * 4, 0);
      }
    };
    if (j_begin < j_end) {
      load_rec(P, rr, j_begin, n64 - 1);
      int j = j_begin;
      while (true) {
        load_rec(Q, rr, j + 1, n64 - 1);
        emit(P, j);
        if (++j >= j_end) break;
        load_rec(P, rr, j + 1, n64 - 1);
        emit(Q, j);
        if (++j >= j_end) break;
      }
      if constexpr (HEAD) {
        if (lane == 0) {
#pragma unroll
          for (int s = 0; s < S; ++s)
            if (acc[s]) atomicAdd(&cnt[s * hd.C + cur_c], acc[s]);
        }
      }
    }
  }
  if constexpr (HEAD) {
    __syncthreads();
    for (int t = threadIdx.x; t < S * hd.C; t += blockDim.x) {
      const int s = t / hd.C, c = t % hd.C;
      if (b0 + s < B) hd.logits[(int64_t)(b0 + s) * hd.C + c] = (float)cnt[t] / hd.tau;
    }
  }
}

// Tile and chunk bound of fc_soft_rec_net_kernel for a network (K = 8):
// 4-sample tiles where every width fits LDS four times over, else 2; the
// chunks per wave of the widest layer must fit one of the compiled bounds.
// 0: the kernel does not apply.
struct RecNetShape {
  int S, CPW;
  size_t lds;
};
static RecNetShape rec_net_shape(int64_t IN, int L, const int64_t* out_dim, int K, int C) {
  RecNetShape r{0, 0, 0};
  if (K != 8 || L < 2) return r;
  int64_t maxw = IN, max_out = 0;
  for (int l = 0; l < L; ++l) {
    maxw = std::max<int64_t>(maxw, out_dim[l]);
    if (l + 1 < L) max_out = std::max<int64_t>(max_out, out_dim[l]);
  }
  const int64_t cap = std::min<int64_t>(device_lds_bytes(), 160 * 1024);
  const int waves = kRecNetThreads / 64;
  const int64_t cpw = cdiv(cdiv(max_out, 64), waves);
  for (int s : {4, 2}) {
    const int64_t lds = maxw * s * 4 + (int64_t)s * std::max(C, 0) * 4;
    if (lds > cap) continue;
    const int bound = s == 4 ? (cpw <= 12 ? 12 : (cpw <= 20 ? 20 : 0))
                             : (cpw <= 16 ? 16 : (cpw <= 32 ? 32 : 0));
    if (bound == 0) continue;
    r.S = s;
    r.CPW = bound;
    r.lds = (size_t)lds;
    return r;
  }
  return r;
}

template <int NODE, int S, int CPW, bool HEAD>
static int launch_rec_net(const float* x, int64_t B, int64_t IN, const RecNetDesc& d, float* y,
                          int maxw, const HeadArgs& hd, size_t lds, hipStream_t st) {
  auto kern = fc_soft_rec_net_kernel<NODE, 8, S, CPW, HEAD>;
  static const size_t static_lds = [&] {
    hipFuncAttributes fa{};
    return hipFuncGetAttributes(&fa, (const void*)kern) == hipSuccess ? fa.sharedSizeBytes
                                                                        : (size_t)-1;
  }();
  SLG_REQUIRE(static_lds == 0, SLG_E_UNSUPPORTED,
              "fc_soft_rec_net: the kernel expects its LDS tile at address 0");
  if (lds > 65536) {
    hipError_t e = hipFuncSetAttribute((const void*)kern,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) {
      set_error("fc_soft_rec_net: cannot reserve %zu B LDS: %s", lds, hipGetErrorString(e));
      return (int)e;
    }
  }
  hipLaunchKernelGGL(kern, dim3((unsigned)cdiv(B, S)), dim3(kRecNetThreads), lds, st, x, (int)B,
                     (int)IN, d, y, maxw, hd);
  SLG_LAUNCH_CHECK("fc_soft_rec_net");
  return 0;
}

template <int NODE, bool HEAD>
static int rec_net_node(const RecNetShape& sh, const float* x, int64_t B, int64_t IN,
                        const RecNetDesc& d, float* y, int maxw, const HeadArgs& hd,
                        hipStream_t st) {
  if (sh.S == 4 && sh.CPW == 12) return launch_rec_net<NODE, 4, 12, HEAD>(x, B, IN, d, y, maxw, hd, sh.lds, st);
  if (sh.S == 4) return launch_rec_net<NODE, 4, 20, HEAD>(x, B, IN, d, y, maxw, hd, sh.lds, st);
  if (sh.CPW == 16) return launch_rec_net<NODE, 2, 16, HEAD>(x, B, IN, d, y, maxw, hd, sh.lds, st);
  return launch_rec_net<NODE, 2, 32, HEAD>(x, B, IN, d, y, maxw, hd, sh.lds, st);
}

// LDS bytes of fc_soft_net_kernel for the widths, or 0 when they do not fit.
static int64_t soft_net_lds(int64_t IN, int L, const int64_t* out_dim, int C) {
  int64_t maxw = IN;
  for (int l = 0; l < L; ++l) maxw = std::max<int64_t>(maxw, out_dim[l]);
  const int64_t bytes = 2 * maxw * 16 + (int64_t)4 * std::max(C, 0) * 4;
  return bytes <= std::min<int64_t>(device_lds_bytes(), 160 * 1024) ? bytes : 0;
}

template <int NODE, int KC, bool HEAD>
static int launch_soft_net(const float* x, int64_t B, int64_t IN, const SoftNetDesc& d, float* y,
                           const HeadArgs& hd, size_t lds, hipStream_t st) {
  auto kern = fc_soft_net_kernel<NODE, KC, HEAD>;
  if (lds > 65536) {
    hipError_t e = hipFuncSetAttribute((const void*)kern,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) {
      set_error("fc_soft_net: cannot reserve %zu B LDS: %s", lds, hipGetErrorString(e));
      return (int)e;
    }
  }
  hipLaunchKernelGGL(kern, dim3((unsigned)cdiv(B, 4)), dim3(kNetSoftThreads), lds, st, x, (int)B,
                     (int)IN, d, y, hd);
  SLG_LAUNCH_CHECK("fc_soft_net");
  return 0;
}

template <int NODE, bool HEAD>
static int soft_net_node(const float* x, int64_t B, int64_t IN, const SoftNetDesc& d, float* y,
                         const HeadArgs& hd, size_t lds, hipStream_t st) {
  if (d.K == 8) return launch_soft_net<NODE, 8, HEAD>(x, B, IN, d, y, hd, lds, st);
  return launch_soft_net<NODE, 0, HEAD>(x, B, IN, d, y, hd, lds, st);
}

// ---------------------------------------------------------------------------
// Inputs wider than LDS: slab staging
// ---------------------------------------------------------------------------
// A workgroup owns 4 samples and one output per thread. The rows are staged
// slab by slab (SL inputs at a time, transposed as in fc_soft_kernel: one
// 16-byte slot per input holds the 4 samples); every thread keeps the
// gathered operand vectors of its output's 2K candidates in registers,
// filling those that fall in the current slab, and after the last slab
// accumulates them in candidate order: the fmaf sequence of fc_soft_kernel,
// so the same bits. The rows are read once per workgroup, so ceil(OUT /
// threads) times per tile: a path for widths the one-pass kernels cannot
// stage, not a fast one.
template <int NODE, int KC, bool REC>
__global__ void __launch_bounds__(KC > 0 ? 1024 : 512)
fc_soft_wide_kernel(const float* __restrict__ x, int B, int IN, int OUT, int Kr, ParamView pv,
                    float inv_tau, float* __restrict__ y, int SL) {
  constexpr int S = 4;
  constexpr int KM = KC > 0 ? KC : 16;
  extern __shared__ __align__(16) unsigned char smem[];
  f32x4* lds = reinterpret_cast<f32x4*>(smem);
  const int K = KC > 0 ? KC : Kr;
  const int b0 = blockIdx.x * S;
  const int rows = min(S, B - b0);
  const int o = blockIdx.y * blockDim.x + threadIdx.x;
  const bool valid = o < OUT;
  FcParams<KM> P;
  load_params<KC, KM, REC>(P, min(o, OUT - 1), K, pv);
  const uint32_t lim = (uint32_t)IN - 1u;
  f32x4 xa[KM], xb[KM];
#pragma unroll
  for (int k = 0; k < KM; ++k) {
    xa[k] = f32x4{0.f, 0.f, 0.f, 0.f};
    xb[k] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  for (int s0 = 0; s0 < IN; s0 += SL) {
    const int sl = min(SL, IN - s0);
    __syncthreads();  // the previous slab's reads are done
    for (int i = threadIdx.x; i < sl; i += blockDim.x) {
      float e[S];
#pragma unroll
      for (int v = 0; v < S; ++v)
        e[v] = (v < rows) ? __builtin_nontemporal_load(x + (int64_t)(b0 + v) * IN + s0 + i) : 0.f;
      lds[i] = f32x4{e[0], e[1], e[2], e[3]};
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < KM; ++k) {
      if (KC > 0 || k < K) {
        const uint32_t ra = min((uint32_t)P.ia[k], lim) - (uint32_t)s0;
        const uint32_t rb = min((uint32_t)P.ib[k], lim) - (uint32_t)s0;
        if (ra < (uint32_t)sl) xa[k] = lds[ra];
        if (rb < (uint32_t)sl) xb[k] = lds[rb];
      }
    }
  }
  f32x4 A = zero_vec<f32x4>(), Bv = zero_vec<f32x4>();
#pragma unroll
  for (int k = 0; k < KM; ++k)
    if (KC > 0 || k < K) fma_acc(A, P.fa[k], xa[k]);
#pragma unroll
  for (int k = 0; k < KM; ++k)
    if (KC > 0 || k < K) fma_acc(Bv, P.fb[k], xb[k]);
  if (valid) {
#pragma unroll
    for (int v = 0; v < S; ++v)
      if (v < rows) y[(int64_t)(b0 + v) * OUT + o] = node_eval<NODE>(A[v], Bv[v], P.p, inv_tau);
  }
}

struct SoftArgs {
  const float* x; int64_t B, IN, OUT; int K;
  ParamView pv;
  float inv_tau; float* y;
  int S, threads;
  HeadArgs hd;  // hd.logits != nullptr: fused GroupSum, y unused
};

// Output chunks per sample tile: enough workgroups to fill the chip twice
// over (at the LDS-limited occupancy) where the tiles fill it less than once,
// whole 64-output wave runs per chunk.
static void soft_grid(const SoftArgs& a, int64_t* n_chunks_out, int64_t* chunk_out) {
  const int64_t tiles = cdiv(a.B, a.S);
  const size_t lds = (size_t)a.IN * a.S * sizeof(float);
  const int per_cu = (int)std::max<int64_t>(1, (int64_t)device_lds_bytes() / std::max<size_t>(lds, 1));
  const int64_t target = (int64_t)device_cus() * std::min(per_cu, 4) * 2;
  int64_t n_chunks = std::max<int64_t>(1, cdiv(target, tiles));
  // tiles that fill every CU's resident workgroups once take the whole
  // output range, so that the GroupSum head can be fused (config 5's head:
  // 256 two-sample tiles, 20.2 us split in two chunks plus a GroupSum
  // launch, 12.4 us fused)
  if (tiles >= (int64_t)device_cus() * std::min(per_cu, 4)) n_chunks = 1;
  n_chunks = std::min<int64_t>(n_chunks, std::max<int64_t>(1, cdiv(a.OUT, 64)));
  const int64_t chunk = cdiv(cdiv(a.OUT, n_chunks), 64) * 64;
  *n_chunks_out = cdiv(a.OUT, chunk);
  *chunk_out = chunk;
}

template <int NODE, int KC, int S, bool HEAD, bool REC>
static int launch_soft_s(const SoftArgs& a, hipStream_t st) {
  int64_t n_chunks, chunk;
  soft_grid(a, &n_chunks, &chunk);
  SLG_REQUIRE(!HEAD || n_chunks == 1, SLG_E_UNSUPPORTED,
              "fc_soft: fused GroupSum needs one output chunk per tile");
  const int64_t grid = cdiv(a.B, S) * n_chunks;
  SLG_REQUIRE(grid < (1LL << 31), SLG_E_SHAPE, "fc_soft: grid too large");
  SLG_REQUIRE(a.OUT * S * 4 < (1LL << 31), SLG_E_SHAPE, "fc_soft: OUT %lld too large",
              (long long)a.OUT);
  auto kern = fc_soft_kernel<NODE, KC, S, HEAD, REC>;
  const int threads = std::min(a.threads, soft_max_threads<KC, S>());
  const size_t lds = (size_t)a.IN * S * sizeof(float) + (HEAD ? (size_t)S * a.hd.C * 4 : 0);
  if constexpr (REC && (KC == 4 || KC == 8)) {
    auto rk = fc_soft_rec_kernel<NODE, KC, S, HEAD>;
    SLG_REQUIRE(lds <= (size_t)device_lds_bytes(), SLG_E_SHAPE, "fc_soft: %zu B LDS needed", lds);
    static const size_t static_lds = [&] {
      hipFuncAttributes fa{};
      return hipFuncGetAttributes(&fa, (const void*)rk) == hipSuccess ? fa.sharedSizeBytes
                                                                      : (size_t)-1;
    }();
    SLG_REQUIRE(static_lds == 0, SLG_E_UNSUPPORTED,
                "fc_soft: records kernel expects its LDS tile at address 0");
    if (lds > 65536) {
      hipError_t e = hipFuncSetAttribute((const void*)rk,
                                         hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
      if (e != hipSuccess) {
        set_error("fc_soft: cannot reserve %zu B LDS: %s", lds, hipGetErrorString(e));
        return (int)e;
      }
    }
    hipLaunchKernelGGL(rk, dim3((unsigned)grid), dim3(threads), lds, st, a.x, (int)a.B,
                       (int)a.IN, (int)a.OUT, reinterpret_cast<const uint32_t*>(a.pv.rec),
                       a.inv_tau, a.y, (int)n_chunks, (int)chunk, a.hd);
    SLG_LAUNCH_CHECK("fc_soft");
    return 0;
  }
  SLG_REQUIRE(lds <= (size_t)device_lds_bytes(), SLG_E_SHAPE, "fc_soft: %zu B LDS needed", lds);
  if (lds > 65536) {
    hipError_t e = hipFuncSetAttribute((const void*)kern,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) {
      set_error("fc_soft: cannot reserve %zu B LDS: %s", lds, hipGetErrorString(e));
      return (int)e;
    }
  }
  hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(threads), lds, st, a.x, (int)a.B,
                     (int)a.IN, (int)a.OUT, a.K, a.pv, a.inv_tau, a.y, (int)n_chunks, (int)chunk,
                     a.hd);
  SLG_LAUNCH_CHECK("fc_soft");
  return 0;
}

template <int NODE, int KC, bool HEAD, bool REC>
static int launch_soft_k(const SoftArgs& a, hipStream_t st) {
  switch (a.S) {
    case 1: return launch_soft_s<NODE, KC, 1, HEAD, REC>(a, st);
    case 2: return launch_soft_s<NODE, KC, 2, HEAD, REC>(a, st);
    case 4: return launch_soft_s<NODE, KC, 4, HEAD, REC>(a, st);
    case 8: return launch_soft_s<NODE, KC, 8, HEAD, REC>(a, st);
    default: break;
  }
  set_error("fc_soft: unsupported tile_samples %d (1, 2, 4, 8)", a.S);
  return SLG_E_ARG;
}

static bool al16(const void* p) { return ((uintptr_t)p % 16) == 0; }

template <int NODE, bool HEAD>
static int launch_soft_node(const SoftArgs& a, hipStream_t st) {
  const ParamView& v = a.pv;
  if (v.rec) {  // records are 16-byte aligned by construction
    if (a.K == 8) return launch_soft_k<NODE, 8, HEAD, true>(a, st);
    if (a.K == 4) return launch_soft_k<NODE, 4, HEAD, true>(a, st);
    return launch_soft_k<NODE, 0, HEAD, true>(a, st);
  }
  if constexpr (!HEAD) {
    const bool vec = al16(v.ca) && al16(v.cb) && al16(v.wa) && al16(v.wb) &&
                     v.cstride % 4 == 0 && v.wstride % 4 == 0;
    if (a.K == 8 && vec) return launch_soft_k<NODE, 8, false, false>(a, st);
    if (a.K == 4 && vec) return launch_soft_k<NODE, 4, false, false>(a, st);
    return launch_soft_k<NODE, 0, false, false>(a, st);
  }
  set_error("fc_soft: the fused GroupSum takes records");
  return SLG_E_ARG;
}

// Samples per workgroup tile and workgroup size, from a sweep on MI355X
// (B = 4096, OUT = 10000-16380, K = 8): IN = 784 -> 4 samples / 256 threads,
// IN = 4096 -> 8 / 512, IN = 10000 -> 4 / 512, IN = 16380 -> 2 / 512. The
// tile takes the largest power of two <= 8 whose rows fit 160 KB of LDS less
// 1 KB for the fused head's counters (4 for narrow inputs, where more,
// smaller workgroups per CU win).
static int pick_tile(int64_t IN, int requested, int64_t B = INT64_MAX) {
  if (requested > 0) return requested;
  const int64_t cap = std::min<int64_t>(device_lds_bytes(), 160 * 1024) - 1024;
  if (IN <= 1280) return 4;
  // small batches: fewer than two 8-sample tiles per CU leave most of the
  // chip idle, 4-sample tiles double the workgroups (B = 256, IN = 2000:
  // 13.1 -> 8.6 us per layer)
  if (IN * 16 <= cap && B < 16 * (int64_t)device_cus()) return 4;
  for (int s : {8, 4, 2, 1})
    if (IN * s * 4 <= cap) return s;
  return 0;
}

// Workgroup size: 256 threads for tiles of at most 40 KB (several workgroups
// per CU), else 512: with one workgroup per CU, eight waves beat sixteen on
// MI355X (config 2 hidden layer 103.2 -> 99.6 us, config 4 walsh layer
// 220.7 -> 203.1 us on records; the array path likewise).
static int pick_threads(int64_t IN, int S, int requested) {
  if (requested > 0) return requested;
  const int64_t lds = IN * S * 4;
  if (lds <= 40 * 1024) return 256;
  return 512;
}

template <int NODE, int KC, bool REC>
static int launch_soft_wide(const SoftArgs& a, hipStream_t st) {
  auto kern = fc_soft_wide_kernel<NODE, KC, REC>;
  const int threads = KC > 0 ? 1024 : 512;
  const int64_t cap = std::min<int64_t>(device_lds_bytes(), 160 * 1024);
  const int SL = (int)(cap / 16);  // inputs per slab: 16 bytes (4 samples) each
  const size_t lds = (size_t)SL * 16;
  if (lds > 65536) {
    hipError_t e = hipFuncSetAttribute((const void*)kern,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) {
      set_error("fc_soft: cannot reserve %zu B LDS: %s", lds, hipGetErrorString(e));
      return (int)e;
    }
  }
  const int64_t tiles = cdiv(a.B, 4), oblocks = cdiv(a.OUT, threads);
  SLG_REQUIRE(tiles < (1LL << 31) && oblocks < 65536, SLG_E_SHAPE, "fc_soft: grid too large");
  hipLaunchKernelGGL(kern, dim3((unsigned)tiles, (unsigned)oblocks), dim3(threads), lds, st, a.x,
                     (int)a.B, (int)a.IN, (int)a.OUT, a.K, a.pv, a.inv_tau, a.y, SL);
  SLG_LAUNCH_CHECK("fc_soft");
  return 0;
}

template <int NODE>
static int launch_soft_wide_node(const SoftArgs& a, hipStream_t st) {
  const ParamView& v = a.pv;
  if (v.rec) {
    if (a.K == 8) return launch_soft_wide<NODE, 8, true>(a, st);
    if (a.K == 4) return launch_soft_wide<NODE, 4, true>(a, st);
    return launch_soft_wide<NODE, 0, true>(a, st);
  }
  const bool vec = al16(v.ca) && al16(v.cb) && al16(v.wa) && al16(v.wb) &&
                   v.cstride % 4 == 0 && v.wstride % 4 == 0;
  if (a.K == 8 && vec) return launch_soft_wide<NODE, 8, false>(a, st);
  if (a.K == 4 && vec) return launch_soft_wide<NODE, 4, false>(a, st);
  return launch_soft_wide<NODE, 0, false>(a, st);
}

static int fc_soft_wide(const SoftArgs& a, int node_kind, hipStream_t st) {
  switch (node_kind) {
    case SLG_NODE_GATE16: return launch_soft_wide_node<SLG_NODE_GATE16>(a, st);
    case SLG_NODE_WALSH: return launch_soft_wide_node<SLG_NODE_WALSH>(a, st);
    case SLG_NODE_MULTILINEAR2: return launch_soft_wide_node<SLG_NODE_MULTILINEAR2>(a, st);
    default: break;
  }
  set_error("fc_soft: unknown node_kind %d", node_kind);
  return SLG_E_ARG;
}

static int fc_soft_dispatch(SoftArgs a, int node_kind, hipStream_t st) {
  const ParamView& v = a.pv;
  const bool head = a.hd.logits != nullptr;
  SLG_REQUIRE((v.rec || (v.ca && v.cb && v.wa && v.wb && v.np)) &&
                  ((a.x && (a.y || head)) || a.B == 0), SLG_E_ARG, "fc_soft: null pointer");
  SLG_REQUIRE(a.B >= 0 && a.IN > 0 && a.OUT > 0, SLG_E_SHAPE, "fc_soft: bad sizes B=%lld IN=%lld OUT=%lld",
              (long long)a.B, (long long)a.IN, (long long)a.OUT);
  SLG_REQUIRE(a.K >= 1 && a.K <= 16, SLG_E_SHAPE, "fc_soft: K=%d outside 1..16", a.K);
  SLG_REQUIRE(a.B < (1LL << 31) && a.IN < (1LL << 28) && a.OUT < (1LL << 31), SLG_E_SHAPE,
              "fc_soft: sizes exceed 32-bit indexing");
  SLG_REQUIRE(v.rec ? al16(v.rec) : (al16(v.np) && v.npstride % 4 == 0), SLG_E_ARG,
              "fc_soft: node parameters must be 16-byte aligned");
  if (head)
    SLG_REQUIRE(a.hd.C > 0 && a.OUT % a.hd.C == 0 && a.B * a.hd.C < (1LL << 31), SLG_E_SHAPE,
                "fc_soft: OUT=%lld not divisible by C=%d", (long long)a.OUT, a.hd.C);
  if (a.B == 0) return 0;
  if (a.S == 0 && pick_tile(a.IN, 0) == 0) {  // rows wider than LDS: slab staging
    SLG_REQUIRE(!head, SLG_E_UNSUPPORTED, "fc_soft: the fused GroupSum needs IN <= %lld",
                (long long)(device_lds_bytes() / 4));
    return fc_soft_wide(a, node_kind, st);
  }
  a.S = pick_tile(a.IN, a.S, a.B);
  SLG_REQUIRE(a.S > 0 && (int64_t)a.IN * a.S * 4 <= device_lds_bytes(), SLG_E_SHAPE,
              "fc_soft: IN=%lld does not fit LDS", (long long)a.IN);
  a.threads = pick_threads(a.IN, a.S, a.threads);
  SLG_REQUIRE(a.threads % 64 == 0 && a.threads <= 1024, SLG_E_ARG, "fc_soft: threads=%d", a.threads);
  if (head) {
    a.hd.per = (int)(a.OUT / a.hd.C);
    switch (node_kind) {
      case SLG_NODE_GATE16: return launch_soft_node<SLG_NODE_GATE16, true>(a, st);
      case SLG_NODE_WALSH: return launch_soft_node<SLG_NODE_WALSH, true>(a, st);
      case SLG_NODE_MULTILINEAR2: return launch_soft_node<SLG_NODE_MULTILINEAR2, true>(a, st);
      default: break;
    }
  } else {
    switch (node_kind) {
      case SLG_NODE_GATE16: return launch_soft_node<SLG_NODE_GATE16, false>(a, st);
      case SLG_NODE_WALSH: return launch_soft_node<SLG_NODE_WALSH, false>(a, st);
      case SLG_NODE_MULTILINEAR2: return launch_soft_node<SLG_NODE_MULTILINEAR2, false>(a, st);
      default: break;
    }
  }
  set_error("fc_soft: unknown node_kind %d", node_kind);
  return SLG_E_ARG;
}

// ---------------------------------------------------------------------------
// Parameter prep: softmax over K candidates and the 4 node coefficients.
// ---------------------------------------------------------------------------
// silogic/functional.py:24-44 — {1,A,B,AB} coefficients of the 16 gates.
__constant__ float c_basis[16][4] = {
    {0, 0, 0, 0}, {0, 0, 0, 1}, {0, 1, 0, -1}, {0, 1, 0, 0}, {0, 0, 1, -1}, {0, 0, 1, 0},
    {0, 1, 1, -2}, {0, 1, 1, -1}, {1, -1, -1, 1}, {1, -1, -1, 2}, {1, 0, -1, 0},
    {1, 0, -1, 1}, {1, -1, 0, 0}, {1, -1, 0, 1}, {1, 0, 0, -1}, {1, 0, 0, 0}};

// Softmax of conn[0..K) into w[0..K) (connectomes.py:114-119); conn == null
// means fixed wiring (w = 1).
__device__ inline void softmax_k(const float* conn, int K, float* w) {
  if (!conn) {
    for (int k = 0; k < K; ++k) w[k] = 1.0f;
    return;
  }
  float m = conn[0];
  for (int k = 1; k < K; ++k) m = fmaxf(m, conn[k]);
  float sum = 0.f;
  for (int k = 0; k < K; ++k) sum += expf(conn[k] - m);
  for (int k = 0; k < K; ++k) w[k] = expf(conn[k] - m) / sum;
}

// The 4 node coefficients of output o from its raw parameters.
__device__ inline float4 node_param(int node, const float* raw, int o) {
  if (node == SLG_NODE_GATE16) {  // softmax(gate_logits) @ BASIS (nodes.py:82-84)
    const float* g = raw + (int64_t)o * 16;
    float m = g[0];
    for (int i = 1; i < 16; ++i) m = fmaxf(m, g[i]);
    float e[16], sum = 0.f;
    for (int i = 0; i < 16; ++i) { e[i] = expf(g[i] - m); sum += e[i]; }
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    for (int i = 0; i < 16; ++i) {
      const float p = e[i] / sum;
      for (int j = 0; j < 4; ++j) acc[j] += p * c_basis[i][j];
    }
    return make_float4(acc[0], acc[1], acc[2], acc[3]);
  }
  const float* r = raw + (int64_t)o * 4;
  if (node == SLG_NODE_WALSH) {  // nodes.py:138-143
    const float t0 = r[0], t1 = r[1], t2 = r[2], t3 = r[3];
    return make_float4(((t0 - t1) - t2) + t3, 2.0f * (t1 - t3), 2.0f * (t2 - t3), 4.0f * t3);
  }
  return make_float4(sigmoidf_(r[0]), sigmoidf_(r[1]), sigmoidf_(r[2]), sigmoidf_(r[3]));
}

__global__ void fc_soft_prep_kernel(const float* __restrict__ conn, int OUT, int K, int node,
                                    const float* __restrict__ raw, float* __restrict__ w,
                                    float* __restrict__ np) {
  const int o = blockIdx.x * blockDim.x + threadIdx.x;
  if (o >= OUT) return;
  for (int s = 0; s < 2; ++s) {
    const int64_t base = ((int64_t)o * 2 + s) * K;
    softmax_k(conn ? conn + base : nullptr, K, w + base);
  }
  reinterpret_cast<float4*>(np)[o] = node_param(node, raw, o);
}

// Records of several layers in one launch. Output o's record is
// rec_quads(K) quads of 32-bit words: idx_a[k] | idx_b[k] << 16 (clamped into
// [0, IN)) for k < K, w_a[K] w_b[K] (softmax), zeros to a whole quad,
// param[4], in the chunk-major layout
// read by load_params<.., REC = true>; outputs past OUT up to the next
// multiple of 64 repeat output OUT-1. With a gather order (from
// slg_fc_soft_schedule), step t of slot s holds candidate order[o][s][t].
// Each workgroup serves one layer.
constexpr int kMaxRecLayers = 16;
struct RecLayer {
  const int* cand;
  const float* conn;
  const float* raw;
  const uint8_t* order;
  float* rec;
  int in_dim, out_dim, node;
};
struct RecNet {
  RecLayer L[kMaxRecLayers];
  int blk_start[kMaxRecLayers + 1];
  int n, K;
};

__global__ void __launch_bounds__(256) fc_soft_records_kernel(RecNet net) {
  int l = 0;
  while (l + 1 < net.n && (int)blockIdx.x >= net.blk_start[l + 1]) ++l;
  const RecLayer& L = net.L[l];
  const int op = ((int)blockIdx.x - net.blk_start[l]) * blockDim.x + threadIdx.x;  // padded
  const int n_pad = (L.out_dim + 63) & ~63;
  if (op >= n_pad) return;
  const int o = min(op, L.out_dim - 1);
  const int K = net.K;
  const int RQ = rec_quads(K);
  // words are written as integers: an index pair with idx_b >= 32640 is a
  // NaN bit pattern, which a float move could quieten
  uint32_t* base =
      reinterpret_cast<uint32_t*>(L.rec) + ((int64_t)(op >> 6) * RQ * 64 + (op & 63)) * 4;
  auto put = [&](int w, uint32_t v) { base[(w >> 2) * 256 + (w & 3)] = v; };
  const int64_t ca = (int64_t)o * 2 * K, cb = ca + K;  // slot a, slot b
  float wa[16], wb[16];
  softmax_k(L.conn ? L.conn + ca : nullptr, K, wa);
  softmax_k(L.conn ? L.conn + cb : nullptr, K, wb);
  for (int t = 0; t < K; ++t) {
    const int ka = L.order ? min((int)L.order[ca + t], K - 1) : t;
    const int kb = L.order ? min((int)L.order[cb + t], K - 1) : t;
    const uint32_t ia = (uint32_t)min(max(L.cand[ca + ka], 0), L.in_dim - 1);
    const uint32_t ib = (uint32_t)min(max(L.cand[cb + kb], 0), L.in_dim - 1);
    put(t, ia | (ib << 16));
    put(K + t, __float_as_uint(wa[ka]));
    put(2 * K + t, __float_as_uint(wb[kb]));
  }
  for (int w = 3 * K; w < 4 * (RQ - 1); ++w) put(w, 0u);
  const float4 p = node_param(L.node, L.raw, o);
  put(4 * (RQ - 1) + 0, __float_as_uint(p.x));
  put(4 * (RQ - 1) + 1, __float_as_uint(p.y));
  put(4 * (RQ - 1) + 2, __float_as_uint(p.z));
  put(4 * (RQ - 1) + 3, __float_as_uint(p.w));
}

// Bank-aware gather order. The soft kernel gathers one candidate per lane
// and step from the LDS tile, whose slots are 16 B (4 samples), 8 B or 4 B
// wide. gfx950's LDS has 64 four-byte banks and serves a wave's read in
// fixed lane groups, one cycle per group plus one per extra distinct slot of
// a bank class within the group (measured with timed ds_read patterns):
//  * ds_read_b128: four groups of 16 lanes, bank class = slot mod 16; lanes
//    0-31 split by the parity of lane bits 2-4 (lanes 0-3, 12-15, 20-27 and
//    4-11, 16-19, 28-31), lanes 32-63 likewise;
//  * ds_read_b64: lanes 0-31 and 32-63, class = slot mod 32;
//  * ds_read_b32: one group of 64 lanes, class = slot mod 64.
// For each lane group of a 64-output chunk and each slot, this picks the
// step at which each output reads each of its K candidates so that few reads
// of one step share a bank class: starting from index order, rounds of
// pairwise step swaps within an output that lower the sum of squared
// per-step bank counts of the two steps: every output finds its best swap in
// parallel against the round's counts, then the outputs apply theirs in
// order, each re-checked against the counts as they are. One wave serves
// 64 / N groups of one slot, the counts live in LDS and only the applies run
// one output at a time. The sum over k is the same; only the fp32 summation
// order changes.
constexpr int kSchedMaxK = 16;

// Chunk lane of member l of lane group g (N lanes per group, as above).
template <int N>
__device__ inline int sched_lane(int g, int l) {
  if constexpr (N == 16) {
    const int j = l >> 2;  // j-th lane quad of parity g & 1 within its half
    const int quad = 2 * j + ((__popc(j) & 1) ^ (g & 1));
    return (g >> 1) * 32 + quad * 4 + (l & 3);
  } else {
    return g * N + l;
  }
}

template <int N>
__global__ void __launch_bounds__(64) fc_soft_schedule_kernel(const int* __restrict__ cand, int OUT,
                                                              int K, uint8_t* __restrict__ order) {
  constexpr int G = 64 / N;
  __shared__ int cnt[G][kSchedMaxK][N];   // reads of bank b at step t
  __shared__ uint8_t ord[64][kSchedMaxK];  // per lane: candidate read at step t
  __shared__ uint8_t ob[64][kSchedMaxK];   // per lane: its bank
  const int lane = threadIdx.x, g = lane / N, l = lane - g * N;
  const int s = blockIdx.x & 1;
  // the groups of one 64-output chunk (a partial last chunk leaves some
  // members of each group idle)
  const int o = (blockIdx.x >> 1) * 64 + sched_lane<N>(g, l);
  const bool active = o < OUT;
  for (int i = lane; i < G * kSchedMaxK * N; i += 64) (&cnt[0][0][0])[i] = 0;
  __syncthreads();
  // start from index order
  if (active)
    for (int st = 0; st < K; ++st) {
      const int b = cand[((int64_t)o * 2 + s) * K + st] & (N - 1);
      ord[lane][st] = (uint8_t)st;
      ob[lane][st] = (uint8_t)b;
      atomicAdd(&cnt[g][st][b], 1);
    }
  __syncthreads();

  // swap rounds (measured: index order converges within six rounds, to the
  // cost a greedy start reaches, at a third of the time)
  for (int round = 0; round < 6; ++round) {
    int p1 = -1, p2 = -1, pscore = 0;
    if (active) {
      for (int t1 = 0; t1 < K; ++t1) {
        const int b1 = ob[lane][t1];
        for (int t2 = t1 + 1; t2 < K; ++t2) {
          const int b2 = ob[lane][t2];
          if (b1 == b2) continue;
          const int sc = cnt[g][t1][b2] - cnt[g][t1][b1] + cnt[g][t2][b1] - cnt[g][t2][b2] + 2;
          if (sc < pscore) { pscore = sc; p1 = t1; p2 = t2; }
        }
      }
    }
    bool applied = false;
    for (int j = 0; j < N; ++j) {
      if (active && l == j && p1 >= 0) {
        const int b1 = ob[lane][p1], b2 = ob[lane][p2];
        if (cnt[g][p1][b2] - cnt[g][p1][b1] + cnt[g][p2][b1] - cnt[g][p2][b2] + 2 < 0) {
          cnt[g][p1][b1] -= 1;
          cnt[g][p1][b2] += 1;
          cnt[g][p2][b2] -= 1;
          cnt[g][p2][b1] += 1;
          const uint8_t k1 = ord[lane][p1], k2 = ord[lane][p2];
          ord[lane][p1] = k2;
          ord[lane][p2] = k1;
          ob[lane][p1] = (uint8_t)b2;
          ob[lane][p2] = (uint8_t)b1;
          applied = true;
        }
      }
      __syncthreads();
    }
    if (!__syncthreads_or(applied)) break;
  }
  if (active)
    for (int st = 0; st < K; ++st) order[((int64_t)o * 2 + s) * K + st] = ord[lane][st];
}

// ---------------------------------------------------------------------------
// GroupSum (silogic/heads.py:16-45).
// ---------------------------------------------------------------------------
template <typename T, bool STE>
__global__ void __launch_bounds__(256) groupsum_kernel(const T* __restrict__ x, int B, int W, int C,
                                                       float tau, float* __restrict__ logits) {
  // one wave per (sample, class): coalesced reads of the class block, wave sum
  const int task = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (task >= B * C) return;
  const int b = task / C, c = task % C;
  const int G = W / C;
  const T* row = x + (int64_t)b * W + (int64_t)c * G;
  float part = 0.f;
  for (int j = lane; j < G; j += 64) {
    const float v = (float)row[j];
    part += STE ? (v > 0.5f ? 1.0f : 0.0f) : v;
  }
  for (int off = 32; off > 0; off >>= 1) part += __shfl_xor(part, off);
  if (lane == 0) logits[task] = part / tau;
}

static ParamView arrays_view(const int32_t* ca, const int32_t* cb, int cstride, const float* wa,
                             const float* wb, int wstride, const float* np) {
  return ParamView{ca, cb, wa, wb, np, cstride, wstride, 4, nullptr};
}

static ParamView records_view(const float* rec) {
  return ParamView{nullptr, nullptr, nullptr, nullptr, nullptr, 0, 0, 0, rec};
}

}  // namespace slg

using namespace slg;

extern "C" {

int slg_fc_soft_fwd(const float* x, int64_t B, int64_t IN, int64_t OUT, int32_t K,
                    const int32_t* cand, const float* w, int32_t node_kind,
                    const float* node_param, float inv_tau, float* out, int32_t tile_samples,
                    int32_t threads, slg_stream_t stream) {
  SLG_REQUIRE(cand && w, SLG_E_ARG, "fc_soft_fwd: null cand/w");
  SoftArgs a{x, B, IN, OUT, K, arrays_view(cand, cand + K, 2 * K, w, w + K, 2 * K, node_param),
             inv_tau, out, tile_samples, threads, HeadArgs{nullptr, 0, 0, 1.0f}};
  return fc_soft_dispatch(a, node_kind, as_stream(stream));
}

int slg_dense_logic_fwd(const float* x, int64_t B, int64_t IN, int64_t OUT, int32_t K,
                        const int32_t* ca, const int32_t* cb, const float* wa, const float* wb,
                        const float* coef, float* out, slg_stream_t stream) {
  SoftArgs a{x, B, IN, OUT, K, arrays_view(ca, cb, K, wa, wb, K, coef), 1.0f, out, 0, 0,
             HeadArgs{nullptr, 0, 0, 1.0f}};
  return fc_soft_dispatch(a, SLG_NODE_GATE16, as_stream(stream));
}

int slg_warp_logic_fwd(const float* x, int64_t B, int64_t IN, int64_t OUT, int32_t K,
                       const int32_t* ca, const int32_t* cb, const float* wa, const float* wb,
                       const float* coef, float inv_tau, float* out, slg_stream_t stream) {
  SoftArgs a{x, B, IN, OUT, K, arrays_view(ca, cb, K, wa, wb, K, coef), inv_tau, out, 0, 0,
             HeadArgs{nullptr, 0, 0, 1.0f}};
  return fc_soft_dispatch(a, SLG_NODE_WALSH, as_stream(stream));
}

int slg_fc_soft_prep(const float* conn, int64_t OUT, int32_t K, int32_t node_kind,
                     const float* raw, float* w, float* node_param, slg_stream_t stream) {
  SLG_REQUIRE(raw && w && node_param, SLG_E_ARG, "fc_soft_prep: null pointer");
  SLG_REQUIRE(OUT > 0 && OUT < (1LL << 31) && K >= 1 && K <= 64, SLG_E_SHAPE,
              "fc_soft_prep: bad OUT/K");
  SLG_REQUIRE(node_kind >= 0 && node_kind <= 2, SLG_E_ARG, "fc_soft_prep: node_kind %d", node_kind);
  SLG_REQUIRE(((uintptr_t)node_param % 16) == 0, SLG_E_ARG, "fc_soft_prep: node_param alignment");
  const int th = 256;
  hipLaunchKernelGGL(fc_soft_prep_kernel, dim3((unsigned)cdiv(OUT, th)), dim3(th), 0,
                     as_stream(stream), conn, (int)OUT, K, node_kind, raw, w, node_param);
  SLG_LAUNCH_CHECK("fc_soft_prep");
  return 0;
}

int slg_fc_soft_records(int32_t n_layers, const int32_t* const* cand, const float* const* conn,
                        const float* const* raw, const int64_t* in_dim, const int64_t* out_dim,
                        int32_t K, const int32_t* node_kind, const uint8_t* const* order,
                        float* const* rec, slg_stream_t stream) {
  SLG_REQUIRE(n_layers >= 1 && n_layers <= kMaxRecLayers, SLG_E_SHAPE,
              "fc_soft_records: n_layers=%d outside 1..%d", n_layers, kMaxRecLayers);
  SLG_REQUIRE(cand && conn && raw && in_dim && out_dim && node_kind && rec, SLG_E_ARG,
              "fc_soft_records: null array");
  SLG_REQUIRE(K >= 1 && K <= 16, SLG_E_SHAPE, "fc_soft_records: K=%d outside 1..16", K);
  RecNet net{};
  net.n = n_layers;
  net.K = K;
  const int th = 256;
  int64_t blocks = 0;
  for (int l = 0; l < n_layers; ++l) {
    SLG_REQUIRE(cand[l] && raw[l] && rec[l], SLG_E_ARG, "fc_soft_records: null pointer, layer %d", l);
    SLG_REQUIRE(in_dim[l] > 0 && in_dim[l] < (1LL << 28) && out_dim[l] > 0 &&
                    out_dim[l] < (1LL << 28), SLG_E_SHAPE, "fc_soft_records: bad sizes, layer %d", l);
    // records hold 16-bit input indices (inputs the soft kernels stage in LDS
    // are far narrower)
    SLG_REQUIRE(in_dim[l] <= 65536, SLG_E_UNSUPPORTED,
                "fc_soft_records: in_dim %lld above 65536, layer %d", (long long)in_dim[l], l);
    SLG_REQUIRE(node_kind[l] >= 0 && node_kind[l] <= 2, SLG_E_ARG,
                "fc_soft_records: node_kind %d", node_kind[l]);
    SLG_REQUIRE(((uintptr_t)rec[l] % 16) == 0, SLG_E_ARG, "fc_soft_records: rec alignment");
    net.L[l] = RecLayer{cand[l], conn[l], raw[l], order ? order[l] : nullptr, rec[l],
                        (int)in_dim[l], (int)out_dim[l], node_kind[l]};
    net.blk_start[l] = (int)blocks;
    blocks += cdiv(cdiv(out_dim[l], 64) * 64, th);
  }
  net.blk_start[n_layers] = (int)blocks;
  hipLaunchKernelGGL(fc_soft_records_kernel, dim3((unsigned)blocks), dim3(th), 0,
                     as_stream(stream), net);
  SLG_LAUNCH_CHECK("fc_soft_records");
  return 0;
}

int slg_fc_soft_schedule(const int32_t* cand, int64_t OUT, int32_t K, int64_t IN, uint8_t* order,
                         slg_stream_t stream) {
  SLG_REQUIRE(cand && order, SLG_E_ARG, "fc_soft_schedule: null pointer");
  SLG_REQUIRE(OUT > 0 && OUT < (1LL << 28) && IN > 0 && K >= 1 && K <= 16, SLG_E_SHAPE,
              "fc_soft_schedule: bad sizes");
  const int S = pick_tile(IN, 0);
  const int lanes = S >= 4 ? 16 : (S == 2 ? 32 : 64);
  // one 64-lane workgroup per (64 / lanes groups, slot)
  const unsigned grid = (unsigned)(cdiv(cdiv(OUT, lanes), 64 / lanes) * 2);
  hipStream_t st = as_stream(stream);
  if (lanes == 16)
    hipLaunchKernelGGL(fc_soft_schedule_kernel<16>, dim3(grid), dim3(64), 0, st, cand, (int)OUT, K, order);
  else if (lanes == 32)
    hipLaunchKernelGGL(fc_soft_schedule_kernel<32>, dim3(grid), dim3(64), 0, st, cand, (int)OUT, K, order);
  else
    hipLaunchKernelGGL(fc_soft_schedule_kernel<64>, dim3(grid), dim3(64), 0, st, cand, (int)OUT, K, order);
  SLG_LAUNCH_CHECK("fc_soft_schedule");
  return 0;
}

int slg_fc_soft_fwd_records(const float* x, int64_t B, int64_t IN, int64_t OUT, int32_t K,
                            const float* rec, int64_t rec_in_dim, int32_t node_kind,
                            float inv_tau, float* out, int32_t tile_samples, int32_t threads,
                            slg_stream_t stream) {
  SLG_REQUIRE(rec, SLG_E_ARG, "fc_soft_fwd_records: null rec");
  SLG_REQUIRE(K >= 1 && K <= 16, SLG_E_SHAPE, "fc_soft_fwd_records: K=%d outside 1..16", K);
  // the records' indices lie below rec_in_dim; the kernel stages IN inputs
  SLG_REQUIRE(rec_in_dim > 0 && IN >= rec_in_dim, SLG_E_SHAPE,
              "fc_soft_fwd_records: x has %lld inputs, the records were built for %lld",
              (long long)IN, (long long)rec_in_dim);
  SoftArgs a{x, B, IN, OUT, K, records_view(rec), inv_tau, out, tile_samples, threads,
             HeadArgs{nullptr, 0, 0, 1.0f}};
  return fc_soft_dispatch(a, node_kind, as_stream(stream));
}

// Which whole-network kernel a stack takes: 1 = fc_soft_net_kernel (every
// activation buffer fits LDS twice, a batch below two 8-sample tiles per
// CU: one launch for the network beats a launch per layer); 2 =
// fc_soft_rec_net_kernel (K = 8, a tile of 4 or 2 samples per workgroup
// through every layer, for batches that give every CU a tile); 0 = a
// launch per layer.
static int soft_net_kind(int64_t B, int64_t IN, int L, const int64_t* out_dim, int K, int C) {
  if (soft_net_lds(IN, L, out_dim, C) && B < 16 * (int64_t)device_cus()) return 1;
  const RecNetShape sh = rec_net_shape(IN, L, out_dim, K, C);
  if (sh.S > 0 && cdiv(B, sh.S) >= device_cus()) return 2;
  return 0;
}

int slg_fc_soft_net_supported(int64_t B, int64_t IN, int32_t n_layers, const int64_t* out_dim,
                              int32_t K, int32_t C) {
  if (B <= 0 || B >= (1LL << 31) || IN <= 0 || IN > 65536 || !out_dim || n_layers < 1 ||
      n_layers > kMaxNetLayers || K < 1 || K > 16 || C < 0)
    return 0;
  for (int l = 0; l < n_layers; ++l)
    if (out_dim[l] <= 0 || out_dim[l] > 65536) return 0;
  if (C > 0 && out_dim[n_layers - 1] % C != 0) return 0;
  return soft_net_kind(B, IN, n_layers, out_dim, K, C);
}

int slg_fc_soft_net_records(const float* x, int64_t B, int64_t IN, int32_t n_layers,
                            const float* const* rec, const int64_t* in_dim,
                            const int64_t* out_dim, int32_t K, int32_t node_kind, float inv_tau,
                            int32_t C, float tau, float* out, slg_stream_t stream) {
  SLG_REQUIRE(rec && in_dim && out_dim && (out || B == 0) && (x || B == 0), SLG_E_ARG,
              "fc_soft_net: null pointer");
  SLG_REQUIRE(n_layers >= 1 && n_layers <= kMaxNetLayers, SLG_E_SHAPE, "fc_soft_net: %d layers",
              n_layers);
  SLG_REQUIRE(K >= 1 && K <= 16 && B >= 0 && B < (1LL << 31) && IN > 0 && IN <= 65536 && C >= 0,
              SLG_E_SHAPE, "fc_soft_net: bad sizes");
  SLG_REQUIRE(node_kind >= 0 && node_kind <= 2, SLG_E_ARG, "fc_soft_net: node_kind %d", node_kind);
  SoftNetDesc d{};
  d.L = n_layers;
  d.K = K;
  d.inv_tau = inv_tau;
  int64_t width = IN, maxw = IN;
  for (int l = 0; l < n_layers; ++l) {
    SLG_REQUIRE(rec[l] && ((uintptr_t)rec[l] % 16) == 0, SLG_E_ARG,
                "fc_soft_net: records of layer %d null or misaligned", l);
    SLG_REQUIRE(out_dim[l] > 0 && out_dim[l] <= 65536, SLG_E_SHAPE,
                "fc_soft_net: layer %d width %lld", l, (long long)out_dim[l]);
    // records hold indices below their layer's in_dim: the input must be
    // at least that wide (the layer reads it by index)
    SLG_REQUIRE(in_dim[l] > 0 && in_dim[l] <= width, SLG_E_SHAPE,
                "fc_soft_net: layer %d reads %lld inputs of %lld", l, (long long)in_dim[l],
                (long long)width);
    d.rec[l] = rec[l];
    d.out_dim[l] = (int)out_dim[l];
    width = out_dim[l];
    maxw = std::max(maxw, width);
  }
  SLG_REQUIRE(C == 0 || out_dim[n_layers - 1] % C == 0, SLG_E_SHAPE,
              "fc_soft_net: last width %lld not divisible by %d classes",
              (long long)out_dim[n_layers - 1], C);
  if (B == 0) return 0;
  const int kind = soft_net_kind(B, IN, n_layers, out_dim, K, C);
  SLG_REQUIRE(kind != 0, SLG_E_UNSUPPORTED,
              "fc_soft_net: no whole-network kernel for these widths and this batch");
  d.maxw = (int)maxw;
  HeadArgs hd{out, C, C > 0 ? (int)(out_dim[n_layers - 1] / C) : 0, tau};
  hipStream_t st = as_stream(stream);
  const bool head = C > 0;
  if (kind == 2) {
    RecNetDesc rd{};
    rd.L = n_layers;
    rd.inv_tau = inv_tau;
    for (int l = 0; l < n_layers; ++l) {
      rd.rec[l] = reinterpret_cast<const uint32_t*>(rec[l]);
      rd.out_dim[l] = (int)out_dim[l];
    }
    const RecNetShape sh = rec_net_shape(IN, n_layers, out_dim, K, C);
    switch (node_kind) {
      case SLG_NODE_GATE16:
        return head ? rec_net_node<SLG_NODE_GATE16, true>(sh, x, B, IN, rd, nullptr, (int)maxw, hd, st)
                    : rec_net_node<SLG_NODE_GATE16, false>(sh, x, B, IN, rd, out, (int)maxw, hd, st);
      case SLG_NODE_WALSH:
        return head ? rec_net_node<SLG_NODE_WALSH, true>(sh, x, B, IN, rd, nullptr, (int)maxw, hd, st)
                    : rec_net_node<SLG_NODE_WALSH, false>(sh, x, B, IN, rd, out, (int)maxw, hd, st);
      default:
        return head ? rec_net_node<SLG_NODE_MULTILINEAR2, true>(sh, x, B, IN, rd, nullptr, (int)maxw, hd, st)
                    : rec_net_node<SLG_NODE_MULTILINEAR2, false>(sh, x, B, IN, rd, out, (int)maxw, hd,
                                                                 st);
    }
  }
  const int64_t lds = soft_net_lds(IN, n_layers, out_dim, C);
  switch (node_kind) {
    case SLG_NODE_GATE16:
      return head ? soft_net_node<SLG_NODE_GATE16, true>(x, B, IN, d, nullptr, hd, lds, st)
                  : soft_net_node<SLG_NODE_GATE16, false>(x, B, IN, d, out, hd, lds, st);
    case SLG_NODE_WALSH:
      return head ? soft_net_node<SLG_NODE_WALSH, true>(x, B, IN, d, nullptr, hd, lds, st)
                  : soft_net_node<SLG_NODE_WALSH, false>(x, B, IN, d, out, hd, lds, st);
    default:
      return head ? soft_net_node<SLG_NODE_MULTILINEAR2, true>(x, B, IN, d, nullptr, hd, lds, st)
                  : soft_net_node<SLG_NODE_MULTILINEAR2, false>(x, B, IN, d, out, hd, lds, st);
  }
}

int slg_fc_soft_groupsum_supported(int64_t B, int64_t IN, int64_t OUT, int32_t C) {
  if (B <= 0 || IN <= 0 || OUT <= 0 || C <= 0 || OUT % C != 0) return 0;
  if (B >= (1LL << 31) || IN >= (1LL << 28) || OUT >= (1LL << 31)) return 0;
  SoftArgs a{};
  a.B = B; a.IN = IN; a.OUT = OUT;
  a.S = pick_tile(IN, 0, B);
  if (a.S <= 0 || IN * a.S * 4 + (int64_t)a.S * C * 4 > device_lds_bytes()) return 0;
  int64_t n_chunks, chunk;
  soft_grid(a, &n_chunks, &chunk);
  return n_chunks == 1 ? 1 : 0;
}

int slg_fc_soft_fwd_groupsum(const float* x, int64_t B, int64_t IN, int64_t OUT, int32_t K,
                             const float* rec, int64_t rec_in_dim, int32_t node_kind,
                             float inv_tau, int32_t C, float tau, float* logits,
                             slg_stream_t stream) {
  SLG_REQUIRE(rec && (logits || B == 0), SLG_E_ARG, "fc_soft_fwd_groupsum: null pointer");
  SLG_REQUIRE(K >= 1 && K <= 16, SLG_E_SHAPE, "fc_soft_fwd_groupsum: K=%d outside 1..16", K);
  SLG_REQUIRE(rec_in_dim > 0 && IN >= rec_in_dim, SLG_E_SHAPE,
              "fc_soft_fwd_groupsum: x has %lld inputs, the records were built for %lld",
              (long long)IN, (long long)rec_in_dim);
  if (B == 0) return 0;
  SLG_REQUIRE(slg_fc_soft_groupsum_supported(B, IN, OUT, C), SLG_E_UNSUPPORTED,
              "fc_soft_fwd_groupsum: B=%lld IN=%lld OUT=%lld C=%d needs the unfused path",
              (long long)B, (long long)IN, (long long)OUT, C);
  SoftArgs a{x, B, IN, OUT, K, records_view(rec), inv_tau, nullptr, 0, 0,
             HeadArgs{logits, C, 0, tau}};
  return fc_soft_dispatch(a, node_kind, as_stream(stream));
}

int slg_groupsum_soft(const float* x, int64_t B, int64_t W, int32_t C, float tau, int32_t ste,
                      float* logits, slg_stream_t stream) {
  SLG_REQUIRE((x && logits) || B == 0, SLG_E_ARG, "groupsum_soft: null pointer");
  SLG_REQUIRE(B >= 0 && B * C < (1LL << 31) && C > 0 && W > 0 && W % C == 0 && W < (1LL << 31),
              SLG_E_SHAPE, "groupsum_soft: W=%lld not divisible by C=%d", (long long)W, C);
  if (B == 0) return 0;
  const unsigned grid = (unsigned)cdiv(B * C, 4);
  if (ste)
    hipLaunchKernelGGL((groupsum_kernel<float, true>), dim3(grid), dim3(256), 0, as_stream(stream), x,
                       (int)B, (int)W, C, tau, logits);
  else
    hipLaunchKernelGGL((groupsum_kernel<float, false>), dim3(grid), dim3(256), 0, as_stream(stream),
                       x, (int)B, (int)W, C, tau, logits);
  SLG_LAUNCH_CHECK("groupsum_soft");
  return 0;
}

int slg_groupsum_hard(const void* x, int32_t dtype, int64_t B, int64_t W, int32_t C,
                      float* logits, slg_stream_t stream) {
  SLG_REQUIRE((x && logits) || B == 0, SLG_E_ARG, "groupsum_hard: null pointer");
  SLG_REQUIRE(B >= 0 && B * C < (1LL << 31) && C > 0 && W > 0 && W % C == 0 && W < (1LL << 31),
              SLG_E_SHAPE, "groupsum_hard: W=%lld not divisible by C=%d", (long long)W, C);
  if (B == 0) return 0;
  const unsigned grid = (unsigned)cdiv(B * C, 4);
  if (dtype == 1)
    hipLaunchKernelGGL((groupsum_kernel<uint8_t, false>), dim3(grid), dim3(256), 0,
                       as_stream(stream), (const uint8_t*)x, (int)B, (int)W, C, 1.0f, logits);
  else
    hipLaunchKernelGGL((groupsum_kernel<float, false>), dim3(grid), dim3(256), 0,
                       as_stream(stream), (const float*)x, (int)B, (int)W, C, 1.0f, logits);
  SLG_LAUNCH_CHECK("groupsum_hard");
  return 0;
}

}  // extern "C"
