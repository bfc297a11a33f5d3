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

template <int DT>
__global__ __launch_bounds__(64 * kRopeWaves) void rope_kernel(const RopeParams P) {
  using Ch = Chunk<DT>;
  constexpr int EPL = Ch::EPL;
  constexpr int ES = DT == kRopeF32 ? 4 : 2;  // element bytes
  const int lane = threadIdx.x & 63;
  const int wv = uni(threadIdx.x >> 6);
  const int half = P.D / 2;
  const int lpr = half / EPL;   // lanes per row (divides 64)
  const int rpw = 64 / lpr;     // rows per wave pass
  const int col = (lane % lpr) * EPL;
  const int lrow = lane / lpr;
  const int nrows = P.Hq + P.Hk;
  const int n = P.nseq;
  const auto cu = const_space(P.cu);

  float invf[EPL];
#pragma unroll
  for (int e = 0; e < EPL; ++e) invf[e] = rnd<DT>(P.inv_freq[col + e]);

  const int t0 = (blockIdx.x * kRopeWaves + wv) * kRopeTokensPerWave;
  if (t0 >= P.T) return;
  // Largest b with cu[b] <= t0 (b = -1: before the first sequence).
  int lo = -1, hi = n;  // cu[lo] <= t0 < cu[hi], with cu[-1] = -inf, cu[n + 1] = +inf
  if (uni(cu[n]) <= t0) lo = n;
  else
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (uni(cu[mid]) <= t0) lo = mid;
      else hi = mid;
    }
  int b = lo;

  for (int i = 0; i < kRopeTokensPerWave; ++i) {
    const int t = t0 + i;
    if (t >= P.T) break;
    while (b < n && uni(cu[b + 1]) <= t) ++b;
    // inside a sequence: 0 <= b < n (cu[b] <= t < cu[b + 1])
    const bool inside = b >= 0 && b < n;
    float c[EPL], s[EPL];
    if (inside) {
      const float pos = rnd<DT>((float)(t - uni(cu[b])));
#pragma unroll
      for (int e = 0; e < EPL; ++e) {
        const float ang = rnd<DT>(mul_rn(pos, invf[e]));
        float sv, cv;
        sincosf(ang, &sv, &cv);  // the accurate library routine
        c[e] = rnd<DT>(cv);
        s[e] = P.sign * rnd<DT>(sv);
      }
    }
    // Four row passes at a time: every load first, then the arithmetic and
    // the stores.
    for (int r0 = lrow; r0 < nrows; r0 += kRopePasses * rpw) {
      Ch x1[kRopePasses], x2[kRopePasses];
      char* dst[kRopePasses];
      bool copy[kRopePasses];
#pragma unroll
      for (int j = 0; j < kRopePasses; ++j) {
        const int r = r0 + j * rpw;
        dst[j] = nullptr;
        if (r < nrows) {
          const bool isq = r < P.Hq;
          const int h = isq ? r : r - P.Hq;
          const char* src = (const char*)(isq ? P.q : P.k) +
                            ((int64_t)t * (isq ? P.q_ss : P.k_ss) +
                             (int64_t)h * (isq ? P.q_sh : P.k_sh)) * ES;
          dst[j] = (char*)(isq ? P.q_out : P.k_out) +
                   ((int64_t)t * (isq ? P.qo_ss : P.ko_ss) +
                    (int64_t)h * (isq ? P.qo_sh : P.ko_sh)) * ES;
          copy[j] = dst[j] != src;
          x1[j].load(src + col * ES);
          x2[j].load(src + (half + col) * ES);
        }
      }
#pragma unroll
      for (int j = 0; j < kRopePasses; ++j) {
        if (!dst[j]) continue;
        if (inside) {
          Ch y1, y2;
#pragma unroll
          for (int e = 0; e < EPL; ++e) {
            y1.v[e] = rnd<DT>(add_rn(rnd<DT>(mul_rn(x1[j].v[e], c[e])),
                                     rnd<DT>(mul_rn(-x2[j].v[e], s[e]))));
            y2.v[e] = rnd<DT>(add_rn(rnd<DT>(mul_rn(x2[j].v[e], c[e])),
                                     rnd<DT>(mul_rn(x1[j].v[e], s[e]))));
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

}  // namespace

hipError_t launch_rope(const RopeParams& P, hipStream_t s) {
  if (P.T <= 0 || P.Hq + P.Hk <= 0) return hipSuccess;
  const int per_block = kRopeWaves * kRopeTokensPerWave;
  const dim3 grid((P.T + per_block - 1) / per_block), block(64 * kRopeWaves);
  switch (P.dtype) {
    case kRopeBF16: hipLaunchKernelGGL(rope_kernel<kRopeBF16>, grid, block, 0, s, P); break;
    case kRopeF16: hipLaunchKernelGGL(rope_kernel<kRopeF16>, grid, block, 0, s, P); break;
    case kRopeF32: hipLaunchKernelGGL(rope_kernel<kRopeF32>, grid, block, 0, s, P); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace fna2
