// fna2_sched.hip — device-built work lists for the varlen kernels.
//
// A varlen launch has one workgroup (or, for the persistent dK/dV kernel,
// one work item) per (tile, head).  The list of tiles is built on the device
// from cu_seqlens (no host synchronisation), longest-processing-time first
// so that long work starts first.  Grouped lists order sequences by total
// work and keep a sequence's tiles together, its longest tile first:
// consecutive tiles of one head then run at about the same time and, with a
// head count that is a multiple of 8 (tile-major grids with the head
// fastest), on the same XCD, so the K / V rows they share come from HBM
// once and from that XCD's L2 after.  Ungrouped lists order every tile by
// its own work.  The reference instead launches a
// (cdiv(max_seqlen, BLOCK), H, N) grid whose out-of-range programs exit at
// once (FNA2/flash_naylis_attn.py:257-259, :784).
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

// Zero the gradient rows of token t if it lies outside [cu[0], cu[N])
// (every token, without sequences: cu may then be null).
__device__ void zero_row(const Problem& p, const ZeroRows& z, int t) {
  const bool any = p.nseq > 0;
  const int cq0 = any ? p.cu_q[0] : 0, cqn = any ? p.cu_q[p.nseq] : 0;
  const int ck0 = any ? p.cu_k[0] : 0, ckn = any ? p.cu_k[p.nseq] : 0;
  if (t < p.total_q && (t < cq0 || t >= cqn)) {
    for (int h = 0; h < p.H; ++h) {
      uint16_t* r = (uint16_t*)z.dq.ptr + (int64_t)t * z.dq.ss + (int64_t)h * z.dq.sh;
      for (int d = 0; d < p.D; ++d) r[d] = 0;
    }
    for (int h = 0; h < p.H_G; ++h) {
      uint16_t* r = (uint16_t*)z.drq.ptr + (int64_t)t * z.drq.ss + (int64_t)h * z.drq.sh;
      for (int d = 0; d < p.R; ++d) r[d] = 0;
    }
  }
  if (t < p.total_k && (t < ck0 || t >= ckn)) {
    for (int h = 0; h < p.H_KV; ++h) {
      uint16_t* r = (uint16_t*)z.dk.ptr + (int64_t)t * z.dk.ss + (int64_t)h * z.dk.sh;
      uint16_t* s = (uint16_t*)z.dv.ptr + (int64_t)t * z.dv.ss + (int64_t)h * z.dv.sh;
      for (int d = 0; d < p.D; ++d) r[d] = 0, s[d] = 0;
    }
    for (int h = 0; h < p.H_G; ++h) {
      uint16_t* r = (uint16_t*)z.drk.ptr + (int64_t)t * z.drk.ss + (int64_t)h * z.drk.sh;
      for (int d = 0; d < p.R; ++d) r[d] = 0;
    }
  }
}

__global__ __launch_bounds__(kThreads) void build_tiles_kernel(Problem p, TileList la,
                                                               TileList lb, int nlists,
                                                               ZeroRows zero) {
  if ((int)blockIdx.x >= nlists) {
    const int t = ((int)blockIdx.x - nlists) * kThreads + (int)threadIdx.x;
    if (t < zero.rows) zero_row(p, zero, t);
    return;
  }
  const TileList& L = blockIdx.x == 0 ? la : lb;
  const TileSpec spec = L.spec;
  TileRec* __restrict__ tiles = L.tiles;
  int* __restrict__ count = L.count;
  const int cap = L.cap;
  constexpr int nbuckets = kMaxBuckets;
  __shared__ int hist[kMaxBuckets];
  __shared__ int warp_tot[kThreads / 64];
  const int tid = threadIdx.x;
  for (int i = tid; i < nbuckets; i += kThreads) hist[i] = 0;
  __syncthreads();

  // Buckets: 0 = most work (work past the last bucket ties).  A grouped
  // list buckets whole sequences by their total work, an ungrouped one
  // buckets tiles by their own.  The histogram counts tiles, so its prefix
  // sums are positions.
  auto seq_bucket = [&](const SeqExt& e, int n) {
    int w = 0;
    for (int t = 0; t < n && w < nbuckets; ++t) w += tile_work(e, spec, p.causal, t);
    return nbuckets - 1 - min(w, nbuckets - 1);
  };
  auto tile_bucket = [&](const SeqExt& e, int t) {
    return nbuckets - 1 - min(tile_work(e, spec, p.causal, t), nbuckets - 1);
  };

  // Pass 1: tiles per bucket.
  for (int b = tid; b < p.nseq; b += kThreads) {
    const SeqExt e = seq_ext(p, b);
    const int n = tile_count(e, spec);
    if (n <= 0) continue;
    if (spec.group) {
      atomicAdd(&hist[seq_bucket(e, n)], n);
    } else {
      for (int t = 0; t < n; ++t) atomicAdd(&hist[tile_bucket(e, t)], 1);
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

  // Pass 2: scatter.  The order of the claims inside a bucket varies from
  // run to run; no result does: tiles are independent, each writes its own
  // outputs, and each carries its slot (position in (sequence, tile) order:
  // an exclusive scan of the tile counts over the sequences), by which sums
  // over tiles are indexed.  A grouped sequence claims a run of positions
  // and writes its tiles most work first: under the causal mask the last
  // query tile and the first key tile.
  const bool reverse = spec.kind == 0 && p.causal;
  int carry = 0;  // tiles of the sequences before this chunk
  for (int base = 0; base < p.nseq; base += kThreads) {
    const int b = base + tid;
    SeqExt e{};
    int n = 0;
    if (b < p.nseq) {
      e = seq_ext(p, b);
      n = max(tile_count(e, spec), 0);
    }
    int sc = n;  // wave-level inclusive scan of the counts
    for (int off = 1; off < 64; off <<= 1) {
      const int y = __shfl_up(sc, off);
      if (lane >= off) sc += y;
    }
    __syncthreads();  // the previous readers of warp_tot are done
    if (lane == 63) warp_tot[wid] = sc;
    __syncthreads();
    int before = 0, chunk = 0;
    for (int w = 0; w < kThreads / 64; ++w) {
      if (w < wid) before += warp_tot[w];
      chunk += warp_tot[w];
    }
    const int slot0 = carry + before + sc - n;
    carry += chunk;
    if (n <= 0) continue;
    if (spec.group) {
      const int pos = atomicAdd(&hist[seq_bucket(e, n)], n);
      for (int i = 0; i < n; ++i) {
        const int t = reverse ? n - 1 - i : i;
        if (pos + i < cap) tiles[pos + i] = TileRec{b, t, e.q0, e.lq, e.k0, e.lk, slot0 + t, 0};
      }
    } else {
      for (int t = 0; t < n; ++t) {
        const int pos = atomicAdd(&hist[tile_bucket(e, t)], 1);
        if (pos < cap) tiles[pos] = TileRec{b, t, e.q0, e.lq, e.k0, e.lk, slot0 + t, 0};
      }
    }
  }
}

}  // namespace

hipError_t launch_zero_rows(const Problem& p, const ZeroRows& zero, hipStream_t stream) {
  if (zero.rows <= 0) return hipSuccess;
  const int zblocks = (zero.rows + kThreads - 1) / kThreads;
  const TileList none{{0, 1, 1, 0}, nullptr, nullptr, 0};
  hipLaunchKernelGGL(build_tiles_kernel, dim3(zblocks), dim3(kThreads), 0, stream, p, none,
                     none, 0, zero);
  return hipGetLastError();
}

hipError_t launch_build_tiles(const Problem& p, const TileList& a, const TileList* b,
                              const ZeroRows* zero, hipStream_t stream) {
  const int nlists = b ? 2 : 1;
  ZeroRows z{};
  if (zero) z = *zero;
  const int zblocks = z.rows > 0 ? (z.rows + kThreads - 1) / kThreads : 0;
  hipLaunchKernelGGL(build_tiles_kernel, dim3(nlists + zblocks), dim3(kThreads), 0, stream, p,
                     a, b ? *b : a, nlists, z);
  return hipGetLastError();
}

}  // namespace fna2
