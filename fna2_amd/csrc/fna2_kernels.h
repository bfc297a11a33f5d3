// fna2_kernels.h — kernel parameter blocks and host launch wrappers.
#pragma once

#include "fna2_device.h"

namespace fna2 {

struct FwdParams {
  Problem p;
  TView q, k, v, rq, rk, o, lse;
  const float* gs;
  const TileRec* tiles;  // varlen: device tile list (null in dense mode)
  const int* n_tiles;  // varlen: device tile count
};

struct BwdParams {
  Problem p;
  TView q, k, v, rq, rk, o, lse, dout, delta, dq, dk, dv, drq, drk;
  // Workspace written by the dQ kernel for the dK/dV kernel:
  TView nlse;  // -LSE log2(e), fp32 [H][rows]
  const float* gs;
  float* dgs;            // [H_G]
  float* dgs_partial;    // [query tiles][4 waves][H_G] partial sums of d_gs
  int q_tiles;           // query tiles of the dQ grid (varlen: capacity)
  int k_tiles;           // key tiles (varlen: capacity of the key-tile list)
  const TileRec* tiles_q;  // varlen: query tiles (dQ kernel)
  const int* n_tiles_q;
  const TileRec* tiles_k;  // varlen: key tiles (dK/dV kernel)
  const int* n_tiles_k;
  int zero_uncovered;  // varlen: the dQ kernel's spare workgroups zero the
                       // gradient rows of tokens outside every sequence
};

// Forward tile shape (queries per workgroup / keys per iteration at d = 64;
// d = 128 steps 32 keys at a time).  kFwdBN is also the work unit the
// varlen tile list sorts by.
constexpr int kFwdBM = 128;
constexpr int kFwdBN = 64;
// Backward: the dK/dV kernel tiles keys by kv_bn(D, rank tile) and walks
// queries kKvBM at a time; the dQ kernel tiles queries by kDqBM and walks
// keys kDqBN at a time.  A dK/dV item is four producer waves of kv_kpw
// 32-key slices: two at d = 64 with a rank tile of at most 32 (the rows and
// accumulators of 64 keys fit a wave's registers there, and each block's
// operand reads, DMA and barrier then serve twice the MFMAs), one
// otherwise.
constexpr int kv_kpw(int D, int rpl) { return (D == 64 && rpl <= 32) ? 2 : 1; }
constexpr int kv_bn(int D, int rpl) { return 128 * kv_kpw(D, rpl); }
constexpr int kKvBM = 32;
constexpr int kDqBM = 128;
constexpr int kDqBN = 64;

// Rank padded to a multiple of 32 (the LDS tile width of the rank part of a
// key or query tile): 0, 32 or 64.
inline int padded_rank32(int H_G, int R) {
  return (H_G > 0 && R > 0) ? ((R + 31) / 32) * 32 : 0;
}

// Varlen rotary embedding (fna2_rope.hip).  Element strides; q_out/k_out
// equal q/k (in place) or are disjoint from them.
constexpr int kRopeBF16 = 1, kRopeF16 = 2, kRopeF32 = 3;
struct RopeParams {
  int dtype, T, Hq, Hk, D, nseq, sign;
  const int* cu;         // [nseq + 1]
  const float* inv_freq;  // [D / 2]
  const void* q;
  const void* k;
  void* q_out;  // forward: the rotated rows; backward: dq
  void* k_out;  //                                       dk
  int64_t q_ss, q_sh, k_ss, k_sh, qo_ss, qo_sh, ko_ss, ko_sh;
  const float* wq;  // RMSNorm weights [D] of q / k rows (null: no norm)
  const float* wk;
  float eps;
  // backward of the normalised rotation: incoming gradients, dw partials
  // [2][rope_blocks(T)][D] and the weight gradients
  const void* gq;
  const void* gk;
  int64_t gq_ss, gq_sh, gk_ss, gk_sh;
  float* part;
  float* dwq;
  float* dwk;
};
int rope_blocks(int T);  // workgroups of a rotary launch over T tokens
hipError_t launch_rope(const RopeParams& P, hipStream_t s);
hipError_t launch_rope_norm_bwd(const RopeParams& P, hipStream_t s);

// One-token decode against a KV cache (fna2_decode.hip).  q, rq, o, lse:
// row (b, h) at ptr + b * sb + h * sh; caches: row j of (b, h) at
// ptr + b * sb + h * sh + j * ss.
struct DecodeParams {
  int B, H, H_KV, H_G, D, R, group;
  int nsplit;      // key splits per (sequence, KV head), <= 64
  int split_keys;  // keys per split, a multiple of 32
  int max_len;     // cache rows; lengths are clamped to it
  float c, c2, qa;  // as in Problem
  const int* seqlens;  // [B] valid rows per sequence, or null (all max_len)
  TView q, rq, k, v, rk, o, lse;  // lse.ptr may be null
  const float* gs;
  float* acc;  // nsplit > 1: [nsplit][B][H][D] unnormalised numerators
  float* ml;   // nsplit > 1: [nsplit][B][H] (max, sum) pairs
};
constexpr int kDecodeStages = 2;  // LDS ring depth of a decode wave
// Rank-tile chunks of a decode kernel for `rch` used chunks (graph heads of
// a group x R / 8): 0, 4, 8, 16 or 32; -1 if too wide.
int decode_rank_chunks(int rch);
int decode_stage_bytes(int D, int rc);
hipError_t launch_decode(const DecodeParams& P, int rc, hipStream_t s);
hipError_t launch_decode_merge(const DecodeParams& P, hipStream_t s);

hipError_t launch_fwd(const FwdParams& P, int rp, int grid, hipStream_t s);
hipError_t launch_bwd_dkdv(const BwdParams& P, int rpl, int grid, hipStream_t s);
hipError_t launch_bwd_dq(const BwdParams& P, int rpl, int grid, hipStream_t s);
hipError_t launch_bwd_dgs(const BwdParams& P, hipStream_t s);

// d_gs[h] = sum of the dQ kernel's partials of head h in a fixed order
// (deterministic), by one wave per head: wave w of `nw` takes heads w,
// w + nw, ...  Shared by the reduce kernel and the dK/dV kernel, which does it
// in passing when it runs.
__device__ __forceinline__ void reduce_dgs_waves(const BwdParams& P, int w, int nw, int lane) {
  const int tiles = P.n_tiles_q ? min(*P.n_tiles_q, P.q_tiles) : P.q_tiles;
  const int rows = 4 * tiles, H_G = P.p.H_G;
  for (int h = w; h < H_G; h += nw) {
    float acc = 0.f;
    for (int t = lane; t < rows; t += 64) acc += P.dgs_partial[(int64_t)t * H_G + h];
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off);
    if (lane == 0) P.dgs[h] = acc;
  }
}

}  // namespace fna2
