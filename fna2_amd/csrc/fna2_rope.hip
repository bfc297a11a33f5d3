// fna2_rope.hip — varlen rotary position embedding for gfx950.
//
// Replaces NaylisAttention._apply_rope_varlen, which loops over the packed
// sequences on the host (a .tolist() synchronisation per call) and applies
// RotaryPositionalEmbedding.forward to each (FNA2/attention_fna2.py:620-647,
// :143-170).  Here one launch covers every token: token t of sequence b
// (cu[b] <= t < cu[b+1]) sits at position p = t - cu[b], found on the
// device, and for i < D/2
//     angle_i   = p * inv_freq[i]
//     y_i       = x_i cos(angle_i) - x_{i+D/2} sin(angle_i)
//     y_{i+D/2} = x_{i+D/2} cos(angle_i) + x_i sin(angle_i)
// (rotate_half, :158-161; the cos/sin table repeats the D/2 angles,
// :150-154).  The reference builds the table in the tensor's dtype, so for
// bf16/fp16 the position, inv_freq, the angle, cos and sin are each rounded
// to that dtype, and the products and their sum are rounded as separate
// elementwise ops (:169-170); the kernel rounds at the same points (no
// contraction into fused multiply-adds).  sign = -1 rotates by -angle: the
// gradient of the rotation, with the same rounding as autograd's
// g cos + rotate_half^T(g sin).
//
// HBM-bound: each (token, head) row is read once and written once.  A lane
// owns 16 bytes of the row's first half and the matching 16 bytes of its
// second half; the lanes of a wave cover 64 / LPR rows at a time, and the
// lane keeps the cos/sin of its 16-byte column range for all the token's
// heads (computed once per token).  A workgroup covers 16 consecutive
// tokens (4 per wave); the sequence of a wave's first token comes from a
// binary search of cu_seqlens, later ones by stepping.
#include "fna2_kernels.h"

namespace fna2 {

namespace {

constexpr int kRopeTokensPerWave = 4;
constexpr int kRopeWaves = 4;
constexpr int kRopePasses = 4;  // row passes whose loads are in flight together
constexpr int kBwdPasses = 2;   // (the norm backward holds twice the data per pass)

// Products and sums that are never fused into a multiply-add (the
// reference evaluates them as separate elementwise ops).
__device__ __forceinline__ float mul_rn(float a, float b) {
#pragma clang fp contract(off)
  return a * b;
}
__device__ __forceinline__ float add_rn(float a, float b) {
#pragma clang fp contract(off)
  return a + b;
}

// Rounding to the element type, as a float.
template <int DT>
__device__ __forceinline__ float rnd(float x) {
  if constexpr (DT == kRopeBF16) {
    return bf16_lo(pack_bf16(x, 0.f));
  } else if constexpr (DT == kRopeF16) {
    return (float)(_Float16)x;
  } else {
    return x;
  }
}

// 16 bytes <-> EPL floats.
template <int DT>
struct Chunk {
  static constexpr int EPL = DT == kRopeF32 ? 4 : 8;
  float v[EPL];
  __device__ __forceinline__ void load(const void* p) {
    const u32x4 w = *(const u32x4*)p;
    if constexpr (DT == kRopeF32) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t u = w[i];  // (a vector element is copied out first)
        v[i] = __builtin_bit_cast(float, u);
      }
    } else if constexpr (DT == kRopeBF16) {
#pragma unroll
      for (int i = 0; i < 4; ++i) v[2 * i] = bf16_lo(w[i]), v[2 * i + 1] = bf16_hi(w[i]);
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const _Float16 lo = __builtin_bit_cast(_Float16, (uint16_t)(w[i] & 0xffffu));
        const _Float16 hi = __builtin_bit_cast(_Float16, (uint16_t)(w[i] >> 16));
        v[2 * i] = (float)lo, v[2 * i + 1] = (float)hi;
      }
    }
  }
  __device__ __forceinline__ void store(void* p) const {
    u32x4 w;
    if constexpr (DT == kRopeF32) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float f = v[i];
        w[i] = __builtin_bit_cast(uint32_t, f);
      }
    } else if constexpr (DT == kRopeBF16) {
#pragma unroll
      for (int i = 0; i < 4; ++i) w[i] = pack_bf16(v[2 * i], v[2 * i + 1]);
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        w[i] = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)v[2 * i]) |
               ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)v[2 * i + 1]) << 16);
    }
    *(u32x4*)p = w;
  }
};

// 16 bytes as loaded (EPL elements), unpacked on use: rows in flight cost
// half the registers of their fp32 values.
template <int DT>
struct Raw {
  static constexpr int EPL = Chunk<DT>::EPL;
  u32x4 w;
  __device__ __forceinline__ void load(const void* p) { w = *(const u32x4*)p; }
  __device__ __forceinline__ void store(void* p) const { *(u32x4*)p = w; }
  __device__ __forceinline__ float get(int e) const {
    if constexpr (DT == kRopeF32) {
      return __builtin_bit_cast(float, (uint32_t)w[e]);
    } else if constexpr (DT == kRopeBF16) {
      return (e & 1) ? bf16_hi(w[e >> 1]) : bf16_lo(w[e >> 1]);
    } else {
      const uint32_t u = w[e >> 1];
      return (float)__builtin_bit_cast(_Float16, (uint16_t)((e & 1) ? (u >> 16) : (u & 0xffffu)));
    }
  }
};

// Lane layout and the token -> sequence walk shared by the kernels: lane
// owns columns [col, col + EPL) of both halves of row lrow + j * rpw of a
// token; a wave covers kRopeTokensPerWave consecutive tokens from t0.
template <int DT>
struct RopeLanes {
  static constexpr int EPL = Chunk<DT>::EPL;
  int lane, half, lpr, rpw, col, lrow, nrows, t0, b;
  __device__ __forceinline__ RopeLanes(const RopeParams& P, int wave_id) {
    lane = threadIdx.x & 63;
    half = P.D / 2;
    lpr = half / EPL;  // lanes per row (divides 64)
    rpw = 64 / lpr;    // rows per wave pass
    col = (lane % lpr) * EPL;
    lrow = lane / lpr;
    nrows = P.Hq + P.Hk;
    t0 = wave_id * kRopeTokensPerWave;
    // Largest b with cu[b] <= t0 (b = -1: before the first sequence).
    const auto cu = const_space(P.cu);
    const int n = P.nseq;
    int lo = -1, hi = n;  // cu[lo] <= t0 < cu[hi]
    if (t0 < P.T) {
      if (uni(cu[n]) <= t0) lo = n;
      else
        while (hi - lo > 1) {
          const int mid = (lo + hi) >> 1;
          if (uni(cu[mid]) <= t0) lo = mid;
          else hi = mid;
        }
    }
    b = lo;
  }
  // Step to token t; returns its position, or -1 outside every sequence.
  __device__ __forceinline__ int position(const RopeParams& P, int t) {
    const auto cu = const_space(P.cu);
    while (b < P.nseq && uni(cu[b + 1]) <= t) ++b;
    return (b >= 0 && b < P.nseq) ? t - uni(cu[b]) : -1;
  }
  // Row pointers (q rows first, then k rows).
  __device__ __forceinline__ const char* in_row(const RopeParams& P, const void* q, const void* k,
                                                int64_t qs, int64_t qh, int64_t ks, int64_t kh,
                                                int t, int r) const {
    constexpr int ES = DT == kRopeF32 ? 4 : 2;
    const bool isq = r < P.Hq;
    const int h = isq ? r : r - P.Hq;
    return (const char*)(isq ? q : k) +
           ((int64_t)t * (isq ? qs : ks) + (int64_t)h * (isq ? qh : kh)) * ES;
  }
};

// Sum over the lpr lanes of a row (lanes lrow * lpr .. + lpr - 1); every
// lane of the wave takes part.
__device__ __forceinline__ float row_sum(float v, int lpr) {
  for (int m = 1; m < lpr; m <<= 1) v += __shfl_xor(v, m);
  return v;
}

// Forward.  NORM: q and / or k rows are RMS-normalised first (weights wq /
// wk; a null weight leaves those rows unnormalised), and the chain then runs
// in fp32 with one rounding at the store.
template <int DT, bool NORM>
__global__ __launch_bounds__(64 * kRopeWaves) void rope_kernel(const RopeParams P) {
  using Ch = Chunk<DT>;
  constexpr int EPL = Ch::EPL;
  constexpr int ES = DT == kRopeF32 ? 4 : 2;
  constexpr int TD = NORM ? kRopeF32 : DT;  // type of the table and of the rotation
  RopeLanes<DT> L(P, blockIdx.x * kRopeWaves + uni(threadIdx.x >> 6));
  // (no early return before the weights' barrier: a wave past the last
  // token runs no token iteration below)
  const int col = L.col, half = L.half;

  float invf[EPL];
#pragma unroll
  for (int e = 0; e < EPL; ++e) invf[e] = rnd<TD>(P.inv_freq[col + e]);
  // the norm weights (q, k), in LDS rather than in every lane's registers
  __shared__ float wsh[NORM ? 2 : 1][NORM ? 512 : 1];
  if constexpr (NORM) {
    for (int d = threadIdx.x; d < P.D; d += 64 * kRopeWaves) {
      wsh[0][d] = P.wq ? P.wq[d] : 1.f;
      wsh[1][d] = P.wk ? P.wk[d] : 1.f;
    }
    __syncthreads();
  }
  const float inv_d = 1.f / (float)P.D;

  for (int i = 0; i < kRopeTokensPerWave; ++i) {
    const int t = L.t0 + i;
    if (t >= P.T) break;
    const int p = L.position(P, t);
    const bool inside = p >= 0;
    float c[EPL], s[EPL];
    if (inside) {
      const float pos = rnd<TD>((float)p);
#pragma unroll
      for (int e = 0; e < EPL; ++e) {
        const float ang = rnd<TD>(mul_rn(pos, invf[e]));
        float sv, cv;
        sincosf(ang, &sv, &cv);  // the accurate library routine
        c[e] = rnd<TD>(cv);
        s[e] = P.sign * rnd<TD>(sv);
      }
    }
    // Four row passes at a time: every load first, then the arithmetic and
    // the stores.  (With the norm every lane makes the same passes: the row
    // sums cross lanes.)
    for (int r0 = L.lrow; (NORM ? r0 - L.lrow : r0) < L.nrows; r0 += kRopePasses * L.rpw) {
      Raw<DT> x1[kRopePasses], x2[kRopePasses];
      float rs[kRopePasses];  // the row's RMS factor (0: no norm)
      char* dst[kRopePasses];
      bool copy[kRopePasses], isq[kRopePasses];
#pragma unroll
      for (int j = 0; j < kRopePasses; ++j) {
        const int r = r0 + j * L.rpw;
        dst[j] = nullptr;
        isq[j] = r < P.Hq;
        if (r < L.nrows) {
          const char* src = L.in_row(P, P.q, P.k, P.q_ss, P.q_sh, P.k_ss, P.k_sh, t, r);
          dst[j] = (char*)L.in_row(P, P.q_out, P.k_out, P.qo_ss, P.qo_sh, P.ko_ss, P.ko_sh, t, r);
          copy[j] = dst[j] != src;
          x1[j].load(src + col * ES);
          x2[j].load(src + (half + col) * ES);
        }
      }
#pragma unroll
      for (int j = 0; j < kRopePasses; ++j) rs[j] = 0.f;
      if constexpr (NORM) {
        if (inside) {
          // RMS of each row (every lane joins the cross-lane sums)
#pragma unroll
          for (int j = 0; j < kRopePasses; ++j) {
            float ss = 0.f;
            if (dst[j]) {
#pragma unroll
              for (int e = 0; e < EPL; ++e) {
                const float a = x1[j].get(e), b2 = x2[j].get(e);
                ss += a * a + b2 * b2;
              }
            }
            ss = row_sum(ss, L.lpr);
            const bool has_w = isq[j] ? P.wq != nullptr : P.wk != nullptr;
            if (dst[j] && has_w) rs[j] = rsqrtf(ss * inv_d + P.eps);
          }
        }
      }
#pragma unroll
      for (int j = 0; j < kRopePasses; ++j) {
        if (!dst[j]) continue;
        if (inside) {
          Ch y1, y2;
#pragma unroll
          for (int e = 0; e < EPL; ++e) {
            float a = x1[j].get(e), b2 = x2[j].get(e);
            if (NORM && rs[j] != 0.f) {  // x r w, as (x r) w
              const float* w = wsh[isq[j] ? 0 : 1];
              a = a * rs[j] * w[col + e];
              b2 = b2 * rs[j] * w[half + col + e];
            }
            y1.v[e] = rnd<TD>(add_rn(rnd<TD>(mul_rn(a, c[e])), rnd<TD>(mul_rn(-b2, s[e]))));
            y2.v[e] = rnd<TD>(add_rn(rnd<TD>(mul_rn(b2, c[e])), rnd<TD>(mul_rn(a, s[e]))));
          }
          y1.store(dst[j] + col * ES);
          y2.store(dst[j] + (half + col) * ES);
        } else if (copy[j]) {  // outside every sequence: unchanged
          x1[j].store(dst[j] + col * ES);
          x2[j].store(dst[j] + (half + col) * ES);
        }
      }
    }
  }
}

// Backward of the normalised rotation (fp32 chain, as the forward with a
// norm): g' = R(-angle) dy, then for rows with a weight
//     dx = r (w g') - x r^3 <x, w g'> / D,     dw += x r g'
// (r = rsqrt(mean(x^2) + eps)); rows without one get dx = g'; tokens
// outside every sequence pass dy through.  Each workgroup writes its dw
// partial sums (fixed order) to part[2][gridDim.x][D].
template <int DT>
__global__ __launch_bounds__(64 * kRopeWaves) void rope_norm_bwd_kernel(const RopeParams P) {
  using Ch = Chunk<DT>;
  constexpr int EPL = Ch::EPL;
  constexpr int ES = DT == kRopeF32 ? 4 : 2;
  __shared__ float red[2][kRopeWaves][512];
  const int wv = uni(threadIdx.x >> 6);
  RopeLanes<DT> L(P, blockIdx.x * kRopeWaves + wv);
  const int col = L.col, half = L.half, lane = L.lane;
  float invf[EPL], wq1[EPL], wq2[EPL], wk1[EPL], wk2[EPL];
  float aq1[EPL], aq2[EPL], ak1[EPL], ak2[EPL];  // dw partials of this lane's columns
#pragma unroll
  for (int e = 0; e < EPL; ++e) {
    invf[e] = P.inv_freq[col + e];
    wq1[e] = P.wq ? P.wq[col + e] : 1.f;
    wq2[e] = P.wq ? P.wq[half + col + e] : 1.f;
    wk1[e] = P.wk ? P.wk[col + e] : 1.f;
    wk2[e] = P.wk ? P.wk[half + col + e] : 1.f;
    aq1[e] = aq2[e] = ak1[e] = ak2[e] = 0.f;
  }
  const float inv_d = 1.f / (float)P.D;

  for (int i = 0; i < kRopeTokensPerWave && L.t0 < P.T; ++i) {
    const int t = L.t0 + i;
    if (t >= P.T) break;
    const int p = L.position(P, t);
    const bool inside = p >= 0;
    float c[EPL], s[EPL];
    if (inside) {
      const float pos = (float)p;
#pragma unroll
      for (int e = 0; e < EPL; ++e) {
        float sv, cv;
        sincosf(mul_rn(pos, invf[e]), &sv, &cv);
        c[e] = cv;
        s[e] = P.sign * sv;
      }
    }
    for (int r0 = L.lrow; r0 - L.lrow < L.nrows; r0 += kBwdPasses * L.rpw) {
      Ch x1[kBwdPasses], x2[kBwdPasses], g1[kBwdPasses], g2[kBwdPasses];
      char* dst[kBwdPasses];
      bool isq[kBwdPasses];
#pragma unroll
      for (int j = 0; j < kBwdPasses; ++j) {
        const int r = r0 + j * L.rpw;
        dst[j] = nullptr;
        isq[j] = r < P.Hq;
        if (r < L.nrows) {
          const char* xs = L.in_row(P, P.q, P.k, P.q_ss, P.q_sh, P.k_ss, P.k_sh, t, r);
          const char* gs = L.in_row(P, P.gq, P.gk, P.gq_ss, P.gq_sh, P.gk_ss, P.gk_sh, t, r);
          dst[j] = (char*)L.in_row(P, P.q_out, P.k_out, P.qo_ss, P.qo_sh, P.ko_ss, P.ko_sh, t, r);
          x1[j].load(xs + col * ES);
          x2[j].load(xs + (half + col) * ES);
          g1[j].load(gs + col * ES);
          g2[j].load(gs + (half + col) * ES);
        }
      }
#pragma unroll
      for (int j = 0; j < kBwdPasses; ++j) {
        if (inside) {
          // g' = R(-angle) dy (the transpose of the forward rotation)
#pragma unroll
          for (int e = 0; e < EPL; ++e) {
            const float a = g1[j].v[e], bq = g2[j].v[e];
            g1[j].v[e] = add_rn(mul_rn(a, c[e]), mul_rn(bq, s[e]));
            g2[j].v[e] = add_rn(mul_rn(bq, c[e]), mul_rn(-a, s[e]));
          }
          float ss = 0.f, tw = 0.f;
          if (dst[j]) {
#pragma unroll
            for (int e = 0; e < EPL; ++e) {
              const float w1 = isq[j] ? wq1[e] : wk1[e], w2 = isq[j] ? wq2[e] : wk2[e];
              ss += x1[j].v[e] * x1[j].v[e] + x2[j].v[e] * x2[j].v[e];
              tw += x1[j].v[e] * w1 * g1[j].v[e] + x2[j].v[e] * w2 * g2[j].v[e];
            }
          }
          ss = row_sum(ss, L.lpr);
          tw = row_sum(tw, L.lpr);
          const bool has_w = isq[j] ? P.wq != nullptr : P.wk != nullptr;
          if (dst[j] && has_w) {
            const float rr = rsqrtf(ss * inv_d + P.eps);
            const float k3 = rr * rr * rr * tw * inv_d;
#pragma unroll
            for (int e = 0; e < EPL; ++e) {
              const float w1 = isq[j] ? wq1[e] : wk1[e], w2 = isq[j] ? wq2[e] : wk2[e];
              const float xr1 = x1[j].v[e] * rr, xr2 = x2[j].v[e] * rr;
              if (isq[j]) aq1[e] += xr1 * g1[j].v[e], aq2[e] += xr2 * g2[j].v[e];
              else ak1[e] += xr1 * g1[j].v[e], ak2[e] += xr2 * g2[j].v[e];
              g1[j].v[e] = rr * w1 * g1[j].v[e] - x1[j].v[e] * k3;
              g2[j].v[e] = rr * w2 * g2[j].v[e] - x2[j].v[e] * k3;
            }
          }
        }
        if (dst[j]) {
          g1[j].store(dst[j] + col * ES);
          g2[j].store(dst[j] + (half + col) * ES);
        }
      }
    }
  }

  // dw partials: lanes sharing columns (lane % lpr), then the waves, in a
  // fixed order.
#pragma unroll
  for (int e = 0; e < EPL; ++e) {
    for (int m = L.lpr; m < 64; m <<= 1) {
      aq1[e] += __shfl_xor(aq1[e], m);
      aq2[e] += __shfl_xor(aq2[e], m);
      ak1[e] += __shfl_xor(ak1[e], m);
      ak2[e] += __shfl_xor(ak2[e], m);
    }
  }
  if (lane < L.lpr) {
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
      red[0][wv][col + e] = aq1[e];
      red[0][wv][half + col + e] = aq2[e];
      red[1][wv][col + e] = ak1[e];
      red[1][wv][half + col + e] = ak2[e];
    }
  }
  __syncthreads();
  for (int d = threadIdx.x; d < 2 * P.D; d += 64 * kRopeWaves) {
    const int which = d / P.D, dd = d - which * P.D;
    float v = 0.f;
#pragma unroll
    for (int w = 0; w < kRopeWaves; ++w) v += red[which][w][dd];
    P.part[((int64_t)which * gridDim.x + blockIdx.x) * P.D + dd] = v;
  }
}

// dw = sum over the workgroups' partials, in a fixed order: workgroup x
// takes 64 of the 2 D columns (lane = column); its 16 waves sum interleaved
// rows of partials (coalesced 256-byte rows), then wave 0 adds the 16 sums.
__global__ __launch_bounds__(1024) void rope_dw_reduce_kernel(const RopeParams P, int nblocks) {
  __shared__ float acc[16][64];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int d = blockIdx.x * 64 + lane;  // in [0, 2 D)
  const bool ok = d < 2 * P.D;
  const int which = ok ? d / P.D : 0, dd = ok ? d - which * P.D : 0;
  const float* src = P.part + (int64_t)which * nblocks * P.D + dd;
  float v = 0.f;
  if (ok) {
    int b = wv;
    for (; b + 7 * 16 < nblocks; b += 8 * 16) {  // eight loads in flight
      float t[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) t[u] = src[(int64_t)(b + 16 * u) * P.D];
#pragma unroll
      for (int u = 0; u < 8; ++u) v += t[u];
    }
    for (; b < nblocks; b += 16) v += src[(int64_t)b * P.D];
  }
  acc[wv][lane] = v;
  __syncthreads();
  if (wv == 0 && ok) {
    float s = 0.f;
#pragma unroll
    for (int w = 0; w < 16; ++w) s += acc[w][lane];
    float* out = which == 0 ? P.dwq : P.dwk;
    if (out) out[dd] = s;
  }
}

}  // namespace

int rope_blocks(int T) {
  const int per_block = kRopeWaves * kRopeTokensPerWave;
  return (T + per_block - 1) / per_block;
}

namespace {
template <int DT>
void launch_rope_dt(const RopeParams& P, dim3 grid, dim3 block, hipStream_t s) {
  if (P.wq || P.wk)
    hipLaunchKernelGGL((rope_kernel<DT, true>), grid, block, 0, s, P);
  else
    hipLaunchKernelGGL((rope_kernel<DT, false>), grid, block, 0, s, P);
}
}  // namespace

hipError_t launch_rope(const RopeParams& P, hipStream_t s) {
  if (P.T <= 0 || P.Hq + P.Hk <= 0) return hipSuccess;
  const dim3 grid(rope_blocks(P.T)), block(64 * kRopeWaves);
  switch (P.dtype) {
    case kRopeBF16: launch_rope_dt<kRopeBF16>(P, grid, block, s); break;
    case kRopeF16: launch_rope_dt<kRopeF16>(P, grid, block, s); break;
    case kRopeF32: launch_rope_dt<kRopeF32>(P, grid, block, s); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_rope_norm_bwd(const RopeParams& P, hipStream_t s) {
  if (P.T <= 0 || P.Hq + P.Hk <= 0) return hipSuccess;
  const int nb = rope_blocks(P.T);
  const dim3 grid(nb), block(64 * kRopeWaves);
  switch (P.dtype) {
    case kRopeBF16: hipLaunchKernelGGL(rope_norm_bwd_kernel<kRopeBF16>, grid, block, 0, s, P); break;
    case kRopeF16: hipLaunchKernelGGL(rope_norm_bwd_kernel<kRopeF16>, grid, block, 0, s, P); break;
    case kRopeF32: hipLaunchKernelGGL(rope_norm_bwd_kernel<kRopeF32>, grid, block, 0, s, P); break;
    default: return hipErrorInvalidValue;
  }
  if (hipGetLastError() != hipSuccess) return hipErrorLaunchFailure;
  hipLaunchKernelGGL(rope_dw_reduce_kernel, dim3((2 * P.D + 63) / 64), dim3(1024), 0, s, P, nb);
  return hipGetLastError();
}

}  // namespace fna2
