// fna2_fwd.hip — FlashNaylisAttention-2 forward for gfx950.
//
// Replaces _fna2_fwd_kernel / _fna2_fwd_varlen_kernel
// (FNA2/flash_naylis_attn.py:58-201, :208-349).
//
// One workgroup = 4 waves = 128 queries of one (sequence, head); wave w owns
// queries 32w..32w+31.  Per 64-key step the wave computes the transposed
// score tile S^T = Ka * Qa^T (64 keys x 32 queries) with the augmented
// contraction of width D + RP (bias fused into the same MFMA chain), so the
// accumulator holds one query per lane (lane % 32) and the row softmax needs
// a single cross-lane exchange (lane ^ 32).  The probabilities, rounded to
// bf16, are the B operand of O^T += V^T * P^T straight from the accumulator
// registers; V^T is staged in LDS with its 16-key groups permuted to match.
// K/Rk and V tiles are double-buffered in LDS (one barrier per step); the Q
// operand stays in registers for the whole loop.
#include "fna2_kernels.h"

namespace fna2 {

namespace {

template <int D, int RP>
struct FwdCfg {
  static constexpr int NT = 256;
  static constexpr int BM = kFwdBM;
  static constexpr int BN = kFwdBN;
  static constexpr int DA = D + RP;
  static constexpr int KS = DA / 16;      // 16-deep steps over the augmented width
  static constexpr int KSD = D / 16;      // ... over the head dim only
  static constexpr int KP = DA * 2 + 16;  // K row pitch in LDS (bytes): 16 mod 32 words
  static constexpr int VP = BN * 2 + 16;  // V^T row pitch in LDS (bytes)
  static constexpr int KBYTES = BN * KP;
  static constexpr int VBYTES = D * VP;
  static constexpr int BUF = KBYTES + VBYTES;
  static constexpr int KCH = BN * DA / 8;  // 16-byte chunks of one Ka tile
  static constexpr int KCH_PT = (KCH + NT - 1) / NT;
  static constexpr int VU = (BN / 4) * (D / 8);  // 4-key x 8-feature V units
  static constexpr int VU_PT = (VU + NT - 1) / NT;
};

template <int D, int RP>
__global__ __launch_bounds__(256) void fwd_kernel(const FwdParams P) {
  using C = FwdCfg<D, RP>;
  __shared__ __attribute__((aligned(16))) uint8_t smem[2 * C::BUF];
  const Problem& p = P.p;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int l32 = lane & 31, hl = lane >> 5;
  const int h = blockIdx.x % p.H;
  const int tix = blockIdx.x / p.H;
  int b, qt;
  if (P.tiles) {
    if (tix >= *P.n_tiles) return;
    const int2 t = P.tiles[tix];
    b = t.x;
    qt = t.y;
  } else {
    const int nqt = cdiv(p.sq, C::BM);
    b = tix % p.nseq;
    qt = nqt - 1 - tix / p.nseq;  // longest causal tiles first
  }
  const SeqExt e = seq_ext(p, b);
  const int kvh = h / p.group;
  const bool graph = (RP > 0) && (h < p.H_G);
  const float bh = graph ? P.gs[h] / p.c : 0.f;

  const uint16_t* qb = seq_base<const uint16_t>(P.q, p, b, e.q0, h);
  const uint16_t* kb = seq_base<const uint16_t>(P.k, p, b, e.k0, kvh);
  const uint16_t* vb = seq_base<const uint16_t>(P.v, p, b, e.k0, kvh);
  const uint16_t* rqb = graph ? seq_base<const uint16_t>(P.rq, p, b, e.q0, h) : nullptr;
  const uint16_t* rkb = graph ? seq_base<const uint16_t>(P.rk, p, b, e.k0, h) : nullptr;

  const int qrow = qt * C::BM + wv * 32 + l32;  // this lane's query
  const bool qvalid = qrow < e.lq;
  const int wq0 = qt * C::BM + wv * 32;
  const int wq_last = min(wq0 + 31, e.lq - 1);

  // Q operand: lane holds Qa[qrow][16s + 8*hl + 0..7] for every step s.
  bf16x8 qreg[C::KS];
  {
    const uint32_t qxor = p.qa < 0.f ? 0x80008000u : 0u;
    const uint32_t qand = p.qa == 0.f ? 0u : 0xffffffffu;
    const uint16_t* qr = qb + (int64_t)qrow * P.q.ss;
#pragma unroll
    for (int s = 0; s < C::KSD; ++s) {
      u32x4 v = {0u, 0u, 0u, 0u};
      if (qvalid) v = ld16(qr + 16 * s + 8 * hl);
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = (v[i] & qand) ^ qxor;
      qreg[s] = as_bf16x8(v);
    }
#pragma unroll
    for (int s = C::KSD; s < C::KS; ++s) {
      const int f = 16 * (s - C::KSD) + 8 * hl;
      u32x4 v = {0u, 0u, 0u, 0u};
      if (graph && qvalid && f < p.R)
        v = scale_bf16x8(ld16(rqb + (int64_t)qrow * P.rq.ss + f), bh);
      qreg[s] = as_bf16x8(v);
    }
  }

  int kv_hi = e.lk;
  if (p.causal) kv_hi = min(kv_hi, min(e.lq, (qt + 1) * C::BM));
  const int nkv = cdiv(max(kv_hi, 0), C::BN);

  u32x4 kreg[C::KCH_PT];
  u32x4 vreg[C::VU_PT][4];
  auto gload = [&](int kt) {
    const int kbase = kt * C::BN;
#pragma unroll
    for (int i = 0; i < C::KCH_PT; ++i) {
      const int c = tid + i * C::NT;
      u32x4 val = {0u, 0u, 0u, 0u};
      if (c < C::KCH) {
        const int row = c / (C::DA / 8), col = (c % (C::DA / 8)) * 8;
        const int key = kbase + row;
        if (key < e.lk) {
          if (col < D)
            val = ld16(kb + (int64_t)key * P.k.ss + col);
          else if (graph && col - D < p.R)
            val = ld16(rkb + (int64_t)key * P.rk.ss + (col - D));
        }
      }
      kreg[i] = val;
    }
#pragma unroll
    for (int i = 0; i < C::VU_PT; ++i) {
      const int u = tid + i * C::NT;
      const int kg = u / (D / 8), d0 = (u % (D / 8)) * 8;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int key = kbase + 4 * kg + r;
        u32x4 val = {0u, 0u, 0u, 0u};
        if (u < C::VU && key < e.lk) val = ld16(vb + (int64_t)key * P.v.ss + d0);
        vreg[i][r] = val;
      }
    }
  };
  auto sstore = [&](int buf) {
    uint8_t* kl = smem + buf * C::BUF;
    uint8_t* vl = kl + C::KBYTES;
#pragma unroll
    for (int i = 0; i < C::KCH_PT; ++i) {
      const int c = tid + i * C::NT;
      if (c < C::KCH) {
        const int row = c / (C::DA / 8), col = (c % (C::DA / 8)) * 8;
        st16(kl + row * C::KP + col * 2, kreg[i]);
      }
    }
#pragma unroll
    for (int i = 0; i < C::VU_PT; ++i) {
      const int u = tid + i * C::NT;
      if (u < C::VU) {
        const int kg = u / (D / 8), d0 = (u % (D / 8)) * 8;
        const int j = kg & 3;
        const int pos = 16 * (kg >> 2) + (((j >> 1) & 1) << 2) + ((j & 1) << 3);
#pragma unroll
        for (int q = 0; q < 8; ++q)
          *(u32x2*)(vl + (d0 + q) * C::VP + pos * 2) =
              gather4(vreg[i][0], vreg[i][1], vreg[i][2], vreg[i][3], q);
      }
    }
  };

  f32x16 oacc[D / 32];
#pragma unroll
  for (int d = 0; d < D / 32; ++d) oacc[d] = f32x16{};
  float m_i = kNegInf, l_i = 0.f;

  if (nkv > 0) {
    gload(0);
    sstore(0);
  }
  __syncthreads();

  for (int kt = 0; kt < nkv; ++kt) {
    const int buf = kt & 1;
    const bool more = kt + 1 < nkv;
    if (more) gload(kt + 1);
    const int kbase = kt * C::BN;
    const bool active = (wq0 <= wq_last) && (!p.causal || kbase <= wq_last);
    if (active) {
      const uint8_t* kl = smem + buf * C::BUF;
      const uint8_t* vl = kl + C::KBYTES;
      f32x16 sacc[C::BN / 32];
#pragma unroll
      for (int kb2 = 0; kb2 < C::BN / 32; ++kb2) {
        f32x16 acc = f32x16{};
        const uint8_t* arow = kl + (kb2 * 32 + l32) * C::KP + 16 * hl;
#pragma unroll
        for (int s = 0; s < C::KSD; ++s)
          acc = mfma32(as_bf16x8(ld16(arow + 32 * s)), qreg[s], acc);
        if (graph) {
#pragma unroll
          for (int s = C::KSD; s < C::KS; ++s)
            acc = mfma32(as_bf16x8(ld16(arow + 32 * s)), qreg[s], acc);
        }
        sacc[kb2] = acc;
      }
      const bool need_mask =
          (kbase + C::BN > e.lk) || (p.causal && kbase + C::BN - 1 > wq0);
      if (need_mask) {
#pragma unroll
        for (int kb2 = 0; kb2 < C::BN / 32; ++kb2)
#pragma unroll
          for (int v = 0; v < 16; ++v) {
            const int key = kbase + kb2 * 32 + 8 * (v >> 2) + 4 * hl + (v & 3);
            if (key >= e.lk || (p.causal && key > qrow)) sacc[kb2][v] = kNegInf;
          }
      }
      float mx = kNegInf;
#pragma unroll
      for (int kb2 = 0; kb2 < C::BN / 32; ++kb2)
#pragma unroll
        for (int v = 0; v < 16; ++v) mx = fmaxf(mx, sacc[kb2][v]);
      mx = wave_pair_max(mx);
      const float m_new = fmaxf(m_i, mx);
      const float m_use = (m_new == kNegInf) ? 0.f : m_new;
      const float alpha = __builtin_amdgcn_exp2f((m_i - m_use) * p.c2);
      const float nm = -m_use * p.c2;
      float ls = 0.f;
      bf16x8 pb[C::BN / 16];
#pragma unroll
      for (int kb2 = 0; kb2 < C::BN / 32; ++kb2)
#pragma unroll
        for (int half = 0; half < 2; ++half) {
          u32x4 pk;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int v0 = 8 * half + 2 * i;
            const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[kb2][v0], p.c2, nm));
            const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[kb2][v0 + 1], p.c2, nm));
            ls += p0 + p1;
            pk[i] = pack_bf16(p0, p1);
          }
          pb[kb2 * 2 + half] = as_bf16x8(pk);
        }
      l_i = l_i * alpha + ls;
      m_i = m_new;
#pragma unroll
      for (int d = 0; d < D / 32; ++d) oacc[d] *= alpha;
#pragma unroll
      for (int s = 0; s < C::BN / 16; ++s)
#pragma unroll
        for (int d = 0; d < D / 32; ++d)
          oacc[d] = mfma32(as_bf16x8(ld16(vl + (d * 32 + l32) * C::VP + (16 * s + 8 * hl) * 2)),
                           pb[s], oacc[d]);
    }
    if (more) sstore(buf ^ 1);
    __syncthreads();
  }

  const float l_tot = wave_pair_sum(l_i);
  if (qvalid) {
    const float inv = 1.f / (l_tot + 1e-6f);
    uint16_t* orow = seq_base<uint16_t>(P.o, p, b, e.q0, h) + (int64_t)qrow * P.o.ss;
#pragma unroll
    for (int d = 0; d < D / 32; ++d)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        u32x2 val;
        val[0] = pack_bf16(oacc[d][4 * g] * inv, oacc[d][4 * g + 1] * inv);
        val[1] = pack_bf16(oacc[d][4 * g + 2] * inv, oacc[d][4 * g + 3] * inv);
        *(u32x2*)(orow + d * 32 + 8 * g + 4 * hl) = val;
      }
    if (hl == 0) {
      float* lrow = seq_base<float>(P.lse, p, b, e.q0, h) + (int64_t)qrow * P.lse.ss;
      *lrow = (m_i == kNegInf)
                  ? kNegInf
                  : m_i * p.c + __builtin_amdgcn_logf(l_tot + 1e-6f) * kLn2;
    }
  }
}

template <int D, int RP>
hipError_t launch_fwd_t(const FwdParams& P, int grid, hipStream_t s) {
  hipLaunchKernelGGL((fwd_kernel<D, RP>), dim3(grid), dim3(256), 0, s, P);
  return hipGetLastError();
}

template <int D>
hipError_t launch_fwd_d(const FwdParams& P, int rp, int grid, hipStream_t s) {
  switch (rp) {
    case 0: return launch_fwd_t<D, 0>(P, grid, s);
    case 16: return launch_fwd_t<D, 16>(P, grid, s);
    case 32: return launch_fwd_t<D, 32>(P, grid, s);
    case 48: return launch_fwd_t<D, 48>(P, grid, s);
    case 64: return launch_fwd_t<D, 64>(P, grid, s);
  }
  return hipErrorInvalidValue;
}

}  // namespace

hipError_t launch_fwd(const FwdParams& P, int rp, int grid, hipStream_t s) {
  if (grid <= 0) return hipSuccess;
  switch (P.p.D) {
    case 64: return launch_fwd_d<64>(P, rp, grid, s);
    case 128: return launch_fwd_d<128>(P, rp, grid, s);
  }
  return hipErrorInvalidValue;
}

}  // namespace fna2
