// fna2_sched.hip — device-built work lists for the varlen kernels.
//
// A varlen launch has one workgroup per (tile, head).  The list of tiles is
// built on the device from cu_seqlens (no host synchronisation) and ordered
// longest-first by the number of inner-loop iterations, so that the
// long-running tiles start first (LPT scheduling).  The reference instead
// launches a (cdiv(max_seqlen, BLOCK), H, N) grid whose out-of-range
// programs exit at once (FNA2/flash_naylis_attn.py:257-259, :784).
#include "fna2_sched.h"

namespace fna2 {

namespace {

constexpr int kThreads = 1024;
constexpr int kMaxBuckets = 4096;

__device__ __forceinline__ int tile_count(const SeqExt& e, const TileSpec& s) {
  return s.kind == 0 ? cdiv(e.lq, s.tile) : cdiv(e.lk, s.tile);
}

// Inner-loop iterations of tile t of a sequence (the sort key).
__device__ __forceinline__ int tile_work(const SeqExt& e, const TileSpec& s,
                                         int causal, int t) {
  if (s.kind == 0) {  // query tile, loop over keys
    int hi = e.lk;
    if (causal) hi = min(hi, min(e.lq, (t + 1) * s.tile));
    return cdiv(max(hi, 0), s.step);
  }
  // key tile, loop over queries
  int lo = causal ? (t * s.tile) / s.step : 0;
  return max(cdiv(e.lq, s.step) - lo, 0);
}

__global__ __launch_bounds__(kThreads) void build_tiles_kernel(
    Problem p, TileSpec spec, int nbuckets, TileRec* __restrict__ tiles,
    int* __restrict__ count, int cap) {
  __shared__ int hist[kMaxBuckets];
  __shared__ int warp_tot[kThreads / 64];
  const int tid = threadIdx.x;
  for (int i = tid; i < nbuckets; i += kThreads) hist[i] = 0;
  __syncthreads();

  // Pass 1: histogram of work, bucket 0 = most work.
  for (int b = tid; b < p.nseq; b += kThreads) {
    const SeqExt e = seq_ext(p, b);
    const int n = tile_count(e, spec);
    for (int t = 0; t < n; ++t) {
      int w = min(tile_work(e, spec, p.causal, t), nbuckets - 1);
      atomicAdd(&hist[nbuckets - 1 - w], 1);
    }
  }
  __syncthreads();

  // Exclusive scan of the histogram: each thread owns a contiguous chunk.
  const int per = (nbuckets + kThreads - 1) / kThreads;
  const int lo = tid * per, hi = min(lo + per, nbuckets);
  int local = 0;
  for (int i = lo; i < hi; ++i) local += hist[i];
  // wave-level inclusive scan of `local`
  const int lane = tid & 63, wid = tid >> 6;
  int incl = local;
  for (int off = 1; off < 64; off <<= 1) {
    int y = __shfl_up(incl, off);
    if (lane >= off) incl += y;
  }
  if (lane == 63) warp_tot[wid] = incl;
  __syncthreads();
  int wbase = 0;
  for (int w = 0; w < wid; ++w) wbase += warp_tot[w];
  int run = wbase + incl - local;  // exclusive prefix of this chunk
  for (int i = lo; i < hi; ++i) {
    int c = hist[i];
    hist[i] = run;
    run += c;
  }
  __syncthreads();
  if (tid == 0) {
    int total = 0;
    for (int w = 0; w < kThreads / 64; ++w) total += warp_tot[w];
    *count = min(total, cap);
  }

  // Pass 2: scatter (order inside a bucket is irrelevant: tiles are
  // independent and each writes its own outputs).
  for (int b = tid; b < p.nseq; b += kThreads) {
    const SeqExt e = seq_ext(p, b);
    const int n = tile_count(e, spec);
    for (int t = 0; t < n; ++t) {
      int w = min(tile_work(e, spec, p.causal, t), nbuckets - 1);
      int pos = atomicAdd(&hist[nbuckets - 1 - w], 1);
      if (pos < cap) tiles[pos] = TileRec{b, t, e.q0, e.lq, e.k0, e.lk, 0, 0};
    }
  }
}

}  // namespace

int tile_buckets(int max_iters) {
  int nb = max_iters + 1;
  if (nb < 1) nb = 1;
  return nb > kMaxBuckets ? kMaxBuckets : nb;
}

hipError_t launch_build_tiles(const Problem& p, const TileSpec& spec,
                              int max_iters, TileRec* tiles, int* count, int cap,
                              hipStream_t stream) {
  hipLaunchKernelGGL(build_tiles_kernel, dim3(1), dim3(kThreads), 0, stream, p,
                     spec, tile_buckets(max_iters), tiles, count, cap);
  return hipGetLastError();
}

}  // namespace fna2
