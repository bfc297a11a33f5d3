// fna2_bwd.hip — FlashNaylisAttention-2 backward for gfx950.
//
// This file holds the backward's small kernels; dQ/dRq (which also forms
// delta = sum_d O dO, the reference's _fna2_bwd_preprocess[_varlen]_kernel,
// FNA2/flash_naylis_attn.py:356-382, :900-921) and dK/dV/dRk are in
// fna2_bwd_dq.hip and fna2_bwd_dkdv.hip.
//   zero rows: varlen tokens outside [cu[0], cu[N]) get zero gradients;
//   d_gs:      fixed-order sum of the dQ kernel's per-wave partials.
// Together: no atomics anywhere, bitwise deterministic, no pre-zeroing.
//
// Math, per head, with Qa = [a Q | b Rq], Ka = [K | Rk], S = c Qa Ka^T:
//   P = exp(S - LSE),  dP = dO V^T,  dS = P (dP - delta),  dA = c dS
//   dV = P^T dO,  [dK | dRk] = dA^T Qa,  [dQ/a | dRq/b] = dA Ka,
//   d_gs = sum_i <Rq_i, (dS Rk)_i> = (1/c) sum_i <Rq_i, (dA Rk)_i>.
#include "fna2_kernels.h"

namespace fna2 {

namespace {

// Varlen only: zero the gradient rows of tokens outside [cu[0], cu[N]).
__global__ __launch_bounds__(256) void zero_uncovered_kernel(const BwdParams P, int rows) {
  const Problem& p = P.p;
  const int t = blockIdx.x * 256 + threadIdx.x;
  if (t >= rows) return;
  const int cq0 = p.cu_q[0], cqn = p.cu_q[p.nseq];
  const int ck0 = p.cu_k[0], ckn = p.cu_k[p.nseq];
  if (t < p.total_q && (t < cq0 || t >= cqn)) {
    for (int h = 0; h < p.H; ++h) {
      uint16_t* r = (uint16_t*)P.dq.ptr + (int64_t)t * P.dq.ss + (int64_t)h * P.dq.sh;
      for (int d = 0; d < p.D; ++d) r[d] = 0;
    }
    for (int h = 0; h < p.H_G; ++h) {
      uint16_t* r = (uint16_t*)P.drq.ptr + (int64_t)t * P.drq.ss + (int64_t)h * P.drq.sh;
      for (int d = 0; d < p.R; ++d) r[d] = 0;
    }
  }
  if (t < p.total_k && (t < ck0 || t >= ckn)) {
    for (int h = 0; h < p.H_KV; ++h) {
      uint16_t* r = (uint16_t*)P.dk.ptr + (int64_t)t * P.dk.ss + (int64_t)h * P.dk.sh;
      uint16_t* s = (uint16_t*)P.dv.ptr + (int64_t)t * P.dv.ss + (int64_t)h * P.dv.sh;
      for (int d = 0; d < p.D; ++d) r[d] = 0, s[d] = 0;
    }
    for (int h = 0; h < p.H_G; ++h) {
      uint16_t* r = (uint16_t*)P.drk.ptr + (int64_t)t * P.drk.ss + (int64_t)h * P.drk.sh;
      for (int d = 0; d < p.R; ++d) r[d] = 0;
    }
  }
}

// d_gs[h] = sum of the dQ kernel's per-(query tile, wave) partials of head h,
// in a fixed order (deterministic).  Varlen: the tile count is on the device.
__global__ __launch_bounds__(256) void dgs_reduce_kernel(const float* __restrict__ part,
                                                         int tiles, const int* __restrict__ n_tiles,
                                                         int H_G, float* __restrict__ dgs) {
  __shared__ float red[4];
  const int h = blockIdx.x;
  const int rows = 4 * (n_tiles ? min(*n_tiles, tiles) : tiles);
  float acc = 0.f;
  for (int t = threadIdx.x; t < rows; t += 256) acc += part[(int64_t)t * H_G + h];
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) dgs[h] = (red[0] + red[1]) + (red[2] + red[3]);
}

}  // namespace

hipError_t launch_bwd_zero_uncovered(const BwdParams& P, hipStream_t s) {
  const Problem& p = P.p;
  if (!p.varlen) return hipSuccess;
  const int rows = p.total_q > p.total_k ? p.total_q : p.total_k;
  if (rows <= 0) return hipSuccess;
  hipLaunchKernelGGL(zero_uncovered_kernel, dim3((rows + 255) / 256), dim3(256), 0, s, P, rows);
  return hipGetLastError();
}

hipError_t launch_bwd_dgs(const BwdParams& P, int tiles, hipStream_t s) {
  if (P.p.H_G <= 0) return hipSuccess;
  hipLaunchKernelGGL(dgs_reduce_kernel, dim3(P.p.H_G), dim3(256), 0, s, P.dgs_partial, tiles,
                     P.n_tiles_q, P.p.H_G, P.dgs);
  return hipGetLastError();
}

}  // namespace fna2
