// fna2_bwd.hip — FlashNaylisAttention-2 backward for gfx950.
//
// This file holds the backward's small kernels; dK/dV/dRk and dQ/dRq are in
// fna2_bwd_dkdv.hip and fna2_bwd_dq.hip.
//   pre-pass:  delta = sum_d O dO (replaces _fna2_bwd_preprocess[_varlen]_kernel,
//              FNA2/flash_naylis_attn.py:356-382, :900-921) and the scaled bias
//              operand Rq' = bf16(graph_scale / c * Rq), zero-padded to the
//              kernel's rank width, which the dK/dV kernel streams by DMA;
//   zero rows: varlen tokens outside [cu[0], cu[N]) get zero gradients;
//   d_gs:      fixed-order sum of the dQ kernel's per-workgroup partials.
// Together: no atomics anywhere, bitwise deterministic, no pre-zeroing.
//
// Math, per head, with Qa = [a Q | b Rq], Ka = [K | Rk], S = c Qa Ka^T:
//   P = exp(S - LSE),  dP = dO V^T,  dS = P (dP - delta),  dA = c dS
//   dV = P^T dO,  [dK | dRk] = dA^T Qa,  [dQ/a | dRq/b] = dA Ka,
//   d_gs = sum_i <Rq_i, (dS Rk)_i> = (1/c) sum_i <Rq_i, (dA Rk)_i>.
#include "fna2_kernels.h"

namespace fna2 {

namespace {

// ------------------------------------------------------------- pre-pass ----
// delta[row, h] = sum_d O[row, h, d] * dO[row, h, d]  (fp32), and for graph
// heads Rq'[row, h, 0..rpl) = bf16(b_h * Rq[row, h, 0..R)), zeros past R.
template <int D>
__global__ __launch_bounds__(256) void prep_kernel(const BwdParams P, int64_t nrows, int rpl) {
  const Problem& p = P.p;
  constexpr int G = D / 8;  // lanes per (row, head)
  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int chunk = (int)(gid % G);
  const int64_t rh = gid / G;
  const int h = (int)(rh % p.H);
  const int64_t row = rh / p.H;
  if (row >= nrows) return;  // uniform across the G lanes of a row
  int64_t oo, od, ol, orq, ors;
  if (p.varlen) {
    oo = row * P.o.ss + h * P.o.sh;
    od = row * P.dout.ss + h * P.dout.sh;
    ol = row * P.delta.ss + h * P.delta.sh;
    orq = row * P.rq.ss + h * P.rq.sh;
    ors = row * P.rqs.ss + h * P.rqs.sh;
  } else {
    const int64_t b = row / p.sq, s = row % p.sq;
    oo = b * P.o.sb + s * P.o.ss + h * P.o.sh;
    od = b * P.dout.sb + s * P.dout.ss + h * P.dout.sh;
    ol = b * P.delta.sb + s * P.delta.ss + h * P.delta.sh;
    orq = b * P.rq.sb + s * P.rq.ss + h * P.rq.sh;
    ors = b * P.rqs.sb + s * P.rqs.ss + h * P.rqs.sh;
  }
  if (h < p.H_G && chunk * 8 < rpl) {
    u32x4 r = {0u, 0u, 0u, 0u};
    if (chunk * 8 < p.R) r = ld16((const uint16_t*)P.rq.ptr + orq + chunk * 8);
    st16((uint16_t*)P.rqs.ptr + ors + chunk * 8, scale_bf16x8(r, P.gs[h] / p.c));
  }
  const u32x4 a = ld16((const uint16_t*)P.o.ptr + oo + chunk * 8);
  const u32x4 c = ld16((const uint16_t*)P.dout.ptr + od + chunk * 8);
  float acc = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i)
    acc += bf16_lo(a[i]) * bf16_lo(c[i]) + bf16_hi(a[i]) * bf16_hi(c[i]);
#pragma unroll
  for (int off = G / 2; off > 0; off >>= 1) acc += __shfl_xor(acc, off);
  if (chunk == 0) ((float*)P.delta.ptr)[ol] = acc;
}

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

// d_gs[h] = sum over dQ workgroups of head h (fixed-order tree).
__global__ __launch_bounds__(256) void dgs_reduce_kernel(const float* __restrict__ part,
                                                         int ntiles, int H,
                                                         float* __restrict__ dgs) {
  __shared__ float red[4];
  const int h = blockIdx.x;
  float acc = 0.f;
  for (int t = threadIdx.x; t < ntiles; t += 256) acc += part[(int64_t)t * H + h];
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) dgs[h] = (red[0] + red[1]) + (red[2] + red[3]);
}

}  // namespace

hipError_t launch_bwd_prep(const BwdParams& P, int rpl, hipStream_t s) {
  const Problem& p = P.p;
  const int64_t nrows = p.varlen ? (int64_t)p.total_q : (int64_t)p.nseq * p.sq;
  if (nrows > 0) {
    const int64_t threads = nrows * p.H * (p.D / 8);
    const int64_t grid = (threads + 255) / 256;
    if (p.D == 64)
      hipLaunchKernelGGL((prep_kernel<64>), dim3((unsigned)grid), dim3(256), 0, s, P, nrows, rpl);
    else
      hipLaunchKernelGGL((prep_kernel<128>), dim3((unsigned)grid), dim3(256), 0, s, P, nrows, rpl);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
  }
  if (p.varlen) {
    const int rows = p.total_q > p.total_k ? p.total_q : p.total_k;
    if (rows > 0) {
      hipLaunchKernelGGL(zero_uncovered_kernel, dim3((rows + 255) / 256), dim3(256), 0, s, P, rows);
      return hipGetLastError();
    }
  }
  return hipSuccess;
}

hipError_t launch_bwd_dgs(const BwdParams& P, int nparts, hipStream_t s) {
  if (P.p.H_G <= 0) return hipSuccess;
  hipLaunchKernelGGL(dgs_reduce_kernel, dim3(P.p.H_G), dim3(256), 0, s, P.dgs_partial,
                     nparts / P.p.H, P.p.H, P.dgs);
  return hipGetLastError();
}

}  // namespace fna2
