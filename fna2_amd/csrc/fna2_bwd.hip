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

// d_gs when the dK/dV kernel does not run (no keys): one wave per head.
__global__ __launch_bounds__(64) void dgs_reduce_kernel(const BwdParams P) {
  reduce_dgs_waves(P, blockIdx.x, gridDim.x, threadIdx.x);
}

}  // namespace

hipError_t launch_bwd_dgs(const BwdParams& P, hipStream_t s) {
  if (P.p.H_G <= 0) return hipSuccess;
  hipLaunchKernelGGL(dgs_reduce_kernel, dim3(P.p.H_G), dim3(64), 0, s, P);
  return hipGetLastError();
}

}  // namespace fna2
