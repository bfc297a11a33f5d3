// fna2_bwd.hip — FlashNaylisAttention-2 backward for gfx950.
//
// Replaces the reference's backward kernels
//   delta:     _fna2_bwd_preprocess[_varlen]_kernel (FNA2/flash_naylis_attn.py:356-382, :900-921)
//   dK/dV/dRk: _fna2_bwd_dkdv[_varlen]_kernel       (:390-553, :929-1076)
//   dQ/dRq:    _fna2_bwd_dq[_varlen]_kernel         (:561-693, :1085-1208)
// with four kernels: delta, dK/dV/dRk, dQ/dRq (+ per-workgroup d_gs
// partials) and a fixed-order d_gs reduction.  No atomics: the dK/dV
// workgroup owns its key rows and sums the GQA group's query heads itself,
// so results are bitwise deterministic and no output needs pre-zeroing.
//
// Math, per head, with Qa = [a Q | b Rq], Ka = [K | Rk], S = c Qa Ka^T:
//   P = exp(S - LSE),  dP = dO V^T,  dS = P (dP - delta),  dA = c dS
//   dV = P^T dO,  [dK | dRk] = dA^T Qa,  [dQ/a | dRq/b] = dA Ka,
//   d_gs = sum_i <Rq_i, (dS Rk)_i> = (1/c) sum_i <Rq_i, (dA Rk)_i>.
#include "fna2_kernels.h"

namespace fna2 {

namespace {

// ---------------------------------------------------------------- delta ----
// delta[row, h] = sum_d O[row, h, d] * dO[row, h, d]  (fp32)
template <int D>
__global__ __launch_bounds__(256) void delta_kernel(const BwdParams P, int64_t nrows) {
  const Problem& p = P.p;
  constexpr int G = D / 8;  // lanes per (row, head)
  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int chunk = (int)(gid % G);
  const int64_t rh = gid / G;
  const int h = (int)(rh % p.H);
  const int64_t row = rh / p.H;
  if (row >= nrows) return;  // uniform across the G lanes of a row
  int64_t oo, od, ol;
  if (p.varlen) {
    oo = row * P.o.ss + h * P.o.sh;
    od = row * P.dout.ss + h * P.dout.sh;
    ol = row * P.delta.ss + h * P.delta.sh;
  } else {
    const int64_t b = row / p.sq, s = row % p.sq;
    oo = b * P.o.sb + s * P.o.ss + h * P.o.sh;
    od = b * P.dout.sb + s * P.dout.ss + h * P.dout.sh;
    ol = b * P.delta.sb + s * P.delta.ss + h * P.delta.sh;
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

// Position (in bf16 elements) of rows 4g..4g+3 inside a permuted 32-row block.
__device__ __forceinline__ int perm_group_pos(int g) {
  const int j = g & 3;
  return 16 * (g >> 2) + (((j >> 1) & 1) << 2) + ((j & 1) << 3);
}

// Load a 16-byte chunk of the augmented query row Qa[q][f0..f0+7].
__device__ __forceinline__ u32x4 load_qa(const uint16_t* qrow, const uint16_t* rqrow,
                                         int f0, int D, int R, bool graph, float bh,
                                         uint32_t qand, uint32_t qxor) {
  u32x4 v = {0u, 0u, 0u, 0u};
  if (f0 < D) {
    v = ld16(qrow + f0);
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = (v[i] & qand) ^ qxor;
  } else if (graph && f0 - D < R) {
    v = scale_bf16x8(ld16(rqrow + (f0 - D)), bh);
  }
  return v;
}

// ----------------------------------------------------------- dK / dV ----
template <int D, int RP>
struct KvCfg {
  static constexpr int NT = 256;
  static constexpr int BN = kKvBN;  // keys per workgroup (32 per wave)
  static constexpr int BM = kKvBM;  // queries per step
  static constexpr int DA = D + RP;
  static constexpr int KS = DA / 16;
  static constexpr int KSD = D / 16;
  static constexpr int NFB = (DA + 31) / 32;  // 32-feature blocks of dKa^T
  static constexpr int NDB = D / 32;
  static constexpr int QP = DA * 2 + 16;  // Qa row pitch (bytes)
  static constexpr int OP = D * 2 + 16;   // dO row pitch
  static constexpr int TP = BM * 2 + 16;  // transposed row pitch
  static constexpr int Q_OFF = 0;
  static constexpr int O_OFF = Q_OFF + BM * QP;
  static constexpr int QT_OFF = O_OFF + BM * OP;
  static constexpr int OT_OFF = QT_OFF + NFB * 32 * TP;
  static constexpr int L_OFF = OT_OFF + D * TP;
  static constexpr int BUF = L_OFF + 2 * BM * 4;
  static constexpr int UQ = (BM / 4) * (DA / 8);
  static constexpr int UO = (BM / 4) * (D / 8);
  static constexpr int U_PT = (UQ + UO + NT - 1) / NT;
};

template <int D, int RP>
__global__ __launch_bounds__(256) void dkdv_kernel(const BwdParams P) {
  using C = KvCfg<D, RP>;
  __shared__ __attribute__((aligned(16))) uint8_t smem[2 * C::BUF];
  const Problem& p = P.p;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int l32 = lane & 31, hl = lane >> 5;
  const int kvh = blockIdx.x % p.H_KV;
  const int tix = blockIdx.x / p.H_KV;
  int b, kt;
  if (P.tiles_k) {
    if (tix >= *P.n_tiles_k) return;
    const int2 t = P.tiles_k[tix];
    b = t.x;
    kt = t.y;
  } else {
    b = tix % p.nseq;
    kt = tix / p.nseq;  // causal: low key tiles have the most queries
  }
  const SeqExt e = seq_ext(p, b);
  const int kbase_t = kt * C::BN;
  const int key = kbase_t + wv * 32 + l32;  // this lane's key (column)
  const bool kvalid = key < e.lk;
  const int wk0 = kbase_t + wv * 32;
  const bool wave_has_keys = wk0 < e.lk;

  const uint16_t* kb = seq_base<const uint16_t>(P.k, p, b, e.k0, kvh);
  const uint16_t* vb = seq_base<const uint16_t>(P.v, p, b, e.k0, kvh);

  // Stationary B operands: Ka[key][16s + 8hl + e] and V[key][16s + 8hl + e].
  bf16x8 kreg[C::KS];
  bf16x8 vreg[C::KSD];
#pragma unroll
  for (int s = 0; s < C::KSD; ++s) {
    u32x4 kv = {0u, 0u, 0u, 0u}, vv = {0u, 0u, 0u, 0u};
    if (kvalid) {
      kv = ld16(kb + (int64_t)key * P.k.ss + 16 * s + 8 * hl);
      vv = ld16(vb + (int64_t)key * P.v.ss + 16 * s + 8 * hl);
    }
    kreg[s] = as_bf16x8(kv);
    vreg[s] = as_bf16x8(vv);
  }

  f32x16 dvacc[C::NDB];
  f32x16 dkacc[C::NFB];
#pragma unroll
  for (int i = 0; i < C::NDB; ++i) dvacc[i] = f32x16{};
#pragma unroll
  for (int i = 0; i < C::NFB; ++i) dkacc[i] = f32x16{};

  // Query blocks that can see this key tile.
  const int qb_lo = p.causal ? kbase_t / C::BM : 0;
  const int qb_hi = cdiv(e.lq, C::BM);
  const int nqb = max(qb_hi - qb_lo, 0);
  const uint32_t qxor = p.qa < 0.f ? 0x80008000u : 0u;
  const uint32_t qand = p.qa == 0.f ? 0u : 0xffffffffu;

  for (int hi = 0; hi < p.group; ++hi) {
    const int h = kvh * p.group + hi;
    const bool graph = (RP > 0) && (h < p.H_G);
    const float bh = graph ? P.gs[h] / p.c : 0.f;
    const uint16_t* qb = seq_base<const uint16_t>(P.q, p, b, e.q0, h);
    const uint16_t* ob = seq_base<const uint16_t>(P.dout, p, b, e.q0, h);
    const uint16_t* rqb = graph ? seq_base<const uint16_t>(P.rq, p, b, e.q0, h) : nullptr;
    const float* lb = seq_base<const float>(P.lse, p, b, e.q0, h);
    const float* db = seq_base<const float>(P.delta, p, b, e.q0, h);

    // Bias part of the stationary K operand for this query head.
#pragma unroll
    for (int s = C::KSD; s < C::KS; ++s) {
      const int f = 16 * (s - C::KSD) + 8 * hl;
      u32x4 v = {0u, 0u, 0u, 0u};
      if (graph && kvalid && f < p.R) {
        const uint16_t* rkb = seq_base<const uint16_t>(P.rk, p, b, e.k0, h);
        v = ld16(rkb + (int64_t)key * P.rk.ss + f);
      }
      kreg[s] = as_bf16x8(v);
    }
#pragma unroll
    for (int i = C::NDB; i < C::NFB; ++i) dkacc[i] = f32x16{};

    u32x4 ureg[C::U_PT][4];
    float lreg = 0.f;
    auto gload = [&](int qblk) {
      const int qbase = qblk * C::BM;
#pragma unroll
      for (int i = 0; i < C::U_PT; ++i) {
        const int u = tid + i * C::NT;
#pragma unroll
        for (int r = 0; r < 4; ++r) ureg[i][r] = u32x4{0u, 0u, 0u, 0u};
        if (u < C::UQ) {
          const int rg = u / (C::DA / 8), f0 = (u % (C::DA / 8)) * 8;
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int q = qbase + 4 * rg + r;
            if (q < e.lq)
              ureg[i][r] = load_qa(qb + (int64_t)q * P.q.ss,
                                   graph ? rqb + (int64_t)q * P.rq.ss : nullptr, f0, D,
                                   p.R, graph, bh, qand, qxor);
          }
        } else if (u < C::UQ + C::UO) {
          const int uo = u - C::UQ;
          const int rg = uo / (D / 8), d0 = (uo % (D / 8)) * 8;
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int q = qbase + 4 * rg + r;
            if (q < e.lq) ureg[i][r] = ld16(ob + (int64_t)q * P.dout.ss + d0);
          }
        }
      }
      if (tid < 2 * C::BM) {
        const int q = qbase + (tid & (C::BM - 1));
        lreg = 0.f;
        if (q < e.lq)
          lreg = tid < C::BM ? lb[(int64_t)q * P.lse.ss] * kLog2e : db[(int64_t)q * P.delta.ss];
      }
    };
    auto sstore = [&](int buf) {
      uint8_t* base = smem + buf * C::BUF;
#pragma unroll
      for (int i = 0; i < C::U_PT; ++i) {
        const int u = tid + i * C::NT;
        if (u < C::UQ) {
          const int rg = u / (C::DA / 8), f0 = (u % (C::DA / 8)) * 8;
#pragma unroll
          for (int r = 0; r < 4; ++r)
            st16(base + C::Q_OFF + (4 * rg + r) * C::QP + f0 * 2, ureg[i][r]);
          const int pos = perm_group_pos(rg);
#pragma unroll
          for (int q = 0; q < 8; ++q)
            *(u32x2*)(base + C::QT_OFF + (f0 + q) * C::TP + pos * 2) =
                gather4(ureg[i][0], ureg[i][1], ureg[i][2], ureg[i][3], q);
        } else if (u < C::UQ + C::UO) {
          const int uo = u - C::UQ;
          const int rg = uo / (D / 8), d0 = (uo % (D / 8)) * 8;
#pragma unroll
          for (int r = 0; r < 4; ++r)
            st16(base + C::O_OFF + (4 * rg + r) * C::OP + d0 * 2, ureg[i][r]);
          const int pos = perm_group_pos(rg);
#pragma unroll
          for (int q = 0; q < 8; ++q)
            *(u32x2*)(base + C::OT_OFF + (d0 + q) * C::TP + pos * 2) =
                gather4(ureg[i][0], ureg[i][1], ureg[i][2], ureg[i][3], q);
        }
      }
      if (tid < 2 * C::BM) ((float*)(base + C::L_OFF))[tid] = lreg;
    };

    if (nqb > 0) {
      gload(qb_lo);
      sstore(0);
    }
    __syncthreads();
    for (int it = 0; it < nqb; ++it) {
      const int buf = it & 1;
      const bool more = it + 1 < nqb;
      if (more) gload(qb_lo + it + 1);
      const int qbase = (qb_lo + it) * C::BM;
      const bool active = wave_has_keys && (!p.causal || qbase + C::BM - 1 >= wk0);
      if (active) {
        const uint8_t* base = smem + buf * C::BUF;
        // S = Qa Ka^T: rows = queries, columns = this wave's keys.
        f32x16 sacc = f32x16{};
        const uint8_t* qrow = base + C::Q_OFF + l32 * C::QP + 16 * hl;
#pragma unroll
        for (int s = 0; s < C::KSD; ++s) sacc = mfma32(as_bf16x8(ld16(qrow + 32 * s)), kreg[s], sacc);
        if (graph) {
#pragma unroll
          for (int s = C::KSD; s < C::KS; ++s)
            sacc = mfma32(as_bf16x8(ld16(qrow + 32 * s)), kreg[s], sacc);
        }
        // dP = dO V^T
        f32x16 dpacc = f32x16{};
        const uint8_t* orow = base + C::O_OFF + l32 * C::OP + 16 * hl;
#pragma unroll
        for (int s = 0; s < C::KSD; ++s) dpacc = mfma32(as_bf16x8(ld16(orow + 32 * s)), vreg[s], dpacc);

        const float* lds_l = (const float*)(base + C::L_OFF);
        bf16x8 pb[2], dsb[2];
#pragma unroll
        for (int half = 0; half < 2; ++half) {
          u32x4 pk, dk;
#pragma unroll
          for (int g2 = 0; g2 < 2; ++g2) {
            const int g = 2 * half + g2;  // accumulator registers 4g..4g+3
            const int r0 = 8 * g + 4 * hl;
            const f32x4_t lse4 = *(const f32x4_t*)(lds_l + r0);
            const f32x4_t dl4 = *(const f32x4_t*)(lds_l + C::BM + r0);
            float pv[4], dv[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              const int v = 4 * g + j;
              const int q = qbase + r0 + j;
              const bool ok = q < e.lq && kvalid && (!p.causal || key <= q);
              const float pr = ok ? __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[v], p.c2, -lse4[j])) : 0.f;
              pv[j] = pr;
              dv[j] = p.c * pr * (dpacc[v] - dl4[j]);
            }
            pk[2 * g2] = pack_bf16(pv[0], pv[1]);
            pk[2 * g2 + 1] = pack_bf16(pv[2], pv[3]);
            dk[2 * g2] = pack_bf16(dv[0], dv[1]);
            dk[2 * g2 + 1] = pack_bf16(dv[2], dv[3]);
          }
          pb[half] = as_bf16x8(pk);
          dsb[half] = as_bf16x8(dk);
        }
        // dV^T += dO^T P ; dKa^T += Qa^T dA
#pragma unroll
        for (int s = 0; s < 2; ++s) {
#pragma unroll
          for (int d = 0; d < C::NDB; ++d)
            dvacc[d] = mfma32(
                as_bf16x8(ld16(base + C::OT_OFF + (d * 32 + l32) * C::TP + (16 * s + 8 * hl) * 2)),
                pb[s], dvacc[d]);
#pragma unroll
          for (int f = 0; f < C::NDB; ++f)
            dkacc[f] = mfma32(
                as_bf16x8(ld16(base + C::QT_OFF + (f * 32 + l32) * C::TP + (16 * s + 8 * hl) * 2)),
                dsb[s], dkacc[f]);
          if (graph) {
#pragma unroll
            for (int f = C::NDB; f < C::NFB; ++f)
              dkacc[f] = mfma32(
                  as_bf16x8(ld16(base + C::QT_OFF + (f * 32 + l32) * C::TP + (16 * s + 8 * hl) * 2)),
                  dsb[s], dkacc[f]);
          }
        }
      }
      if (more) sstore(buf ^ 1);
      __syncthreads();
    }

    // dRk for this head (features D..D+R-1 of dKa^T).
    if (graph && kvalid) {
      uint16_t* rrow = seq_base<uint16_t>(P.drk, p, b, e.k0, h) + (int64_t)key * P.drk.ss;
#pragma unroll
      for (int f = C::NDB; f < C::NFB; ++f)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int rf = f * 32 + 8 * g + 4 * hl - D;
          if (rf < p.R) {
            u32x2 val;
            val[0] = pack_bf16(dkacc[f][4 * g], dkacc[f][4 * g + 1]);
            val[1] = pack_bf16(dkacc[f][4 * g + 2], dkacc[f][4 * g + 3]);
            *(u32x2*)(rrow + rf) = val;
          }
        }
    }
  }

  if (kvalid) {
    uint16_t* krow = seq_base<uint16_t>(P.dk, p, b, e.k0, kvh) + (int64_t)key * P.dk.ss;
    uint16_t* vrow = seq_base<uint16_t>(P.dv, p, b, e.k0, kvh) + (int64_t)key * P.dv.ss;
#pragma unroll
    for (int d = 0; d < C::NDB; ++d)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int c0 = d * 32 + 8 * g + 4 * hl;
        u32x2 kv, vv;
        kv[0] = pack_bf16(dkacc[d][4 * g], dkacc[d][4 * g + 1]);
        kv[1] = pack_bf16(dkacc[d][4 * g + 2], dkacc[d][4 * g + 3]);
        vv[0] = pack_bf16(dvacc[d][4 * g], dvacc[d][4 * g + 1]);
        vv[1] = pack_bf16(dvacc[d][4 * g + 2], dvacc[d][4 * g + 3]);
        *(u32x2*)(krow + c0) = kv;
        *(u32x2*)(vrow + c0) = vv;
      }
  }
}

// ----------------------------------------------------------------- dQ ----
template <int D, int RP>
struct DqCfg {
  static constexpr int NT = 256;
  static constexpr int BM = kDqBM;  // queries per workgroup (32 per wave)
  static constexpr int BN = kDqBN;  // keys per step
  static constexpr int DA = D + RP;
  static constexpr int KS = DA / 16;
  static constexpr int KSD = D / 16;
  static constexpr int NFB = (DA + 31) / 32;
  static constexpr int NDB = D / 32;
  static constexpr int KP = DA * 2 + 16;
  static constexpr int VP = D * 2 + 16;
  static constexpr int TP = BN * 2 + 16;
  static constexpr int K_OFF = 0;
  static constexpr int V_OFF = K_OFF + BN * KP;
  static constexpr int KT_OFF = V_OFF + BN * VP;
  static constexpr int BUF = KT_OFF + NFB * 32 * TP;
  static constexpr int UK = (BN / 4) * (DA / 8);
  static constexpr int UV = (BN / 4) * (D / 8);
  static constexpr int U_PT = (UK + UV + NT - 1) / NT;
};

template <int D, int RP>
__global__ __launch_bounds__(256) void dq_kernel(const BwdParams P) {
  using C = DqCfg<D, RP>;
  __shared__ __attribute__((aligned(16))) uint8_t smem[2 * C::BUF];
  __shared__ float red[4];
  const Problem& p = P.p;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int l32 = lane & 31, hl = lane >> 5;
  const int h = blockIdx.x % p.H;
  const int tix = blockIdx.x / p.H;
  int b, qt;
  if (P.tiles_q) {
    if (tix >= *P.n_tiles_q) {
      if (tid == 0) P.dgs_partial[blockIdx.x] = 0.f;
      return;
    }
    const int2 t = P.tiles_q[tix];
    b = t.x;
    qt = t.y;
  } else {
    const int nqt = cdiv(p.sq, C::BM);
    b = tix % p.nseq;
    qt = nqt - 1 - tix / p.nseq;
  }
  const SeqExt e = seq_ext(p, b);
  const int kvh = h / p.group;
  const bool graph = (RP > 0) && (h < p.H_G);
  const float bh = graph ? P.gs[h] / p.c : 0.f;

  const uint16_t* qb = seq_base<const uint16_t>(P.q, p, b, e.q0, h);
  const uint16_t* ob = seq_base<const uint16_t>(P.dout, p, b, e.q0, h);
  const uint16_t* kb = seq_base<const uint16_t>(P.k, p, b, e.k0, kvh);
  const uint16_t* vb = seq_base<const uint16_t>(P.v, p, b, e.k0, kvh);
  const uint16_t* rqb = graph ? seq_base<const uint16_t>(P.rq, p, b, e.q0, h) : nullptr;
  const uint16_t* rkb = graph ? seq_base<const uint16_t>(P.rk, p, b, e.k0, h) : nullptr;

  const int qrow = qt * C::BM + wv * 32 + l32;
  const bool qvalid = qrow < e.lq;
  const int wq0 = qt * C::BM + wv * 32;
  const int wq_last = min(wq0 + 31, e.lq - 1);
  const uint32_t qxor = p.qa < 0.f ? 0x80008000u : 0u;
  const uint32_t qand = p.qa == 0.f ? 0u : 0xffffffffu;

  bf16x8 qreg[C::KS];
  bf16x8 oreg[C::KSD];
  float lse2 = 0.f, dl = 0.f;
  {
    const uint16_t* qr = qb + (int64_t)qrow * P.q.ss;
    const uint16_t* rr = graph ? rqb + (int64_t)qrow * P.rq.ss : nullptr;
#pragma unroll
    for (int s = 0; s < C::KS; ++s) {
      u32x4 v = {0u, 0u, 0u, 0u};
      if (qvalid) v = load_qa(qr, rr, 16 * s + 8 * hl, D, p.R, graph, bh, qand, qxor);
      qreg[s] = as_bf16x8(v);
    }
#pragma unroll
    for (int s = 0; s < C::KSD; ++s) {
      u32x4 v = {0u, 0u, 0u, 0u};
      if (qvalid) v = ld16(ob + (int64_t)qrow * P.dout.ss + 16 * s + 8 * hl);
      oreg[s] = as_bf16x8(v);
    }
    if (qvalid) {
      lse2 = seq_base<const float>(P.lse, p, b, e.q0, h)[(int64_t)qrow * P.lse.ss] * kLog2e;
      dl = seq_base<const float>(P.delta, p, b, e.q0, h)[(int64_t)qrow * P.delta.ss];
    }
  }

  int kv_hi = e.lk;
  if (p.causal) kv_hi = min(kv_hi, min(e.lq, (qt + 1) * C::BM));
  const int nkb = cdiv(max(kv_hi, 0), C::BN);

  u32x4 ureg[C::U_PT][4];
  auto gload = [&](int kblk) {
    const int kbase = kblk * C::BN;
#pragma unroll
    for (int i = 0; i < C::U_PT; ++i) {
      const int u = tid + i * C::NT;
#pragma unroll
      for (int r = 0; r < 4; ++r) ureg[i][r] = u32x4{0u, 0u, 0u, 0u};
      if (u < C::UK) {
        const int rg = u / (C::DA / 8), f0 = (u % (C::DA / 8)) * 8;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int k = kbase + 4 * rg + r;
          if (k < e.lk) {
            if (f0 < D)
              ureg[i][r] = ld16(kb + (int64_t)k * P.k.ss + f0);
            else if (graph && f0 - D < p.R)
              ureg[i][r] = ld16(rkb + (int64_t)k * P.rk.ss + (f0 - D));
          }
        }
      } else if (u < C::UK + C::UV) {
        const int uv = u - C::UK;
        const int rg = uv / (D / 8), d0 = (uv % (D / 8)) * 8;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int k = kbase + 4 * rg + r;
          if (k < e.lk) ureg[i][r] = ld16(vb + (int64_t)k * P.v.ss + d0);
        }
      }
    }
  };
  auto sstore = [&](int buf) {
    uint8_t* base = smem + buf * C::BUF;
#pragma unroll
    for (int i = 0; i < C::U_PT; ++i) {
      const int u = tid + i * C::NT;
      if (u < C::UK) {
        const int rg = u / (C::DA / 8), f0 = (u % (C::DA / 8)) * 8;
#pragma unroll
        for (int r = 0; r < 4; ++r)
          st16(base + C::K_OFF + (4 * rg + r) * C::KP + f0 * 2, ureg[i][r]);
        const int pos = perm_group_pos(rg);
#pragma unroll
        for (int q = 0; q < 8; ++q)
          *(u32x2*)(base + C::KT_OFF + (f0 + q) * C::TP + pos * 2) =
              gather4(ureg[i][0], ureg[i][1], ureg[i][2], ureg[i][3], q);
      } else if (u < C::UK + C::UV) {
        const int uv = u - C::UK;
        const int rg = uv / (D / 8), d0 = (uv % (D / 8)) * 8;
#pragma unroll
        for (int r = 0; r < 4; ++r)
          st16(base + C::V_OFF + (4 * rg + r) * C::VP + d0 * 2, ureg[i][r]);
      }
    }
  };

  f32x16 acc[C::NFB];
#pragma unroll
  for (int i = 0; i < C::NFB; ++i) acc[i] = f32x16{};

  if (nkb > 0) {
    gload(0);
    sstore(0);
  }
  __syncthreads();
  for (int it = 0; it < nkb; ++it) {
    const int buf = it & 1;
    const bool more = it + 1 < nkb;
    if (more) gload(it + 1);
    const int kbase = it * C::BN;
    const bool active = (wq0 <= wq_last) && (!p.causal || kbase <= wq_last);
    if (active) {
      const uint8_t* base = smem + buf * C::BUF;
      // S^T = Ka Qa^T (rows = keys, column = this lane's query)
      f32x16 sacc = f32x16{};
      const uint8_t* krow = base + C::K_OFF + l32 * C::KP + 16 * hl;
#pragma unroll
      for (int s = 0; s < C::KSD; ++s) sacc = mfma32(as_bf16x8(ld16(krow + 32 * s)), qreg[s], sacc);
      if (graph) {
#pragma unroll
        for (int s = C::KSD; s < C::KS; ++s)
          sacc = mfma32(as_bf16x8(ld16(krow + 32 * s)), qreg[s], sacc);
      }
      // dP^T = V dO^T
      f32x16 dpacc = f32x16{};
      const uint8_t* vrow = base + C::V_OFF + l32 * C::VP + 16 * hl;
#pragma unroll
      for (int s = 0; s < C::KSD; ++s) dpacc = mfma32(as_bf16x8(ld16(vrow + 32 * s)), oreg[s], dpacc);

      bf16x8 dsb[2];
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        u32x4 dk;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float dv[2];
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            const int v = 8 * half + 2 * i + j;
            const int k = kbase + 8 * (v >> 2) + 4 * hl + (v & 3);
            const bool ok = qvalid && k < e.lk && (!p.causal || k <= qrow);
            const float pr = ok ? __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[v], p.c2, -lse2)) : 0.f;
            dv[j] = p.c * pr * (dpacc[v] - dl);
          }
          dk[i] = pack_bf16(dv[0], dv[1]);
        }
        dsb[half] = as_bf16x8(dk);
      }
      // dQa^T += Ka^T dA^T
#pragma unroll
      for (int s = 0; s < 2; ++s) {
#pragma unroll
        for (int f = 0; f < C::NDB; ++f)
          acc[f] = mfma32(
              as_bf16x8(ld16(base + C::KT_OFF + (f * 32 + l32) * C::TP + (16 * s + 8 * hl) * 2)),
              dsb[s], acc[f]);
        if (graph) {
#pragma unroll
          for (int f = C::NDB; f < C::NFB; ++f)
            acc[f] = mfma32(
                as_bf16x8(ld16(base + C::KT_OFF + (f * 32 + l32) * C::TP + (16 * s + 8 * hl) * 2)),
                dsb[s], acc[f]);
        }
      }
    }
    if (more) sstore(buf ^ 1);
    __syncthreads();
  }

  float gpart = 0.f;
  if (qvalid) {
    uint16_t* drow = seq_base<uint16_t>(P.dq, p, b, e.q0, h) + (int64_t)qrow * P.dq.ss;
#pragma unroll
    for (int d = 0; d < C::NDB; ++d)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        u32x2 val;
        val[0] = pack_bf16(p.qa * acc[d][4 * g], p.qa * acc[d][4 * g + 1]);
        val[1] = pack_bf16(p.qa * acc[d][4 * g + 2], p.qa * acc[d][4 * g + 3]);
        *(u32x2*)(drow + d * 32 + 8 * g + 4 * hl) = val;
      }
    if (graph) {
      uint16_t* rrow = seq_base<uint16_t>(P.drq, p, b, e.q0, h) + (int64_t)qrow * P.drq.ss;
      const uint16_t* rq = rqb + (int64_t)qrow * P.rq.ss;
#pragma unroll
      for (int f = C::NDB; f < C::NFB; ++f)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int rf = f * 32 + 8 * g + 4 * hl - D;
          if (rf < p.R) {
            const u32x2 rv = *(const u32x2*)(rq + rf);
            gpart += bf16_lo(rv[0]) * acc[f][4 * g] + bf16_hi(rv[0]) * acc[f][4 * g + 1] +
                     bf16_lo(rv[1]) * acc[f][4 * g + 2] + bf16_hi(rv[1]) * acc[f][4 * g + 3];
            u32x2 val;
            val[0] = pack_bf16(bh * acc[f][4 * g], bh * acc[f][4 * g + 1]);
            val[1] = pack_bf16(bh * acc[f][4 * g + 2], bh * acc[f][4 * g + 3]);
            *(u32x2*)(rrow + rf) = val;
          }
        }
    }
  }
  // Workgroup partial of d_gs in a fixed order.
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) gpart += __shfl_xor(gpart, off);
  if (lane == 0) red[wv] = gpart;
  __syncthreads();
  if (tid == 0) P.dgs_partial[blockIdx.x] = ((red[0] + red[1]) + (red[2] + red[3])) / p.c;
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

template <int D, int RP>
hipError_t launch_dkdv_t(const BwdParams& P, int grid, hipStream_t s) {
  hipLaunchKernelGGL((dkdv_kernel<D, RP>), dim3(grid), dim3(256), 0, s, P);
  return hipGetLastError();
}
template <int D, int RP>
hipError_t launch_dq_t(const BwdParams& P, int grid, hipStream_t s) {
  hipLaunchKernelGGL((dq_kernel<D, RP>), dim3(grid), dim3(256), 0, s, P);
  return hipGetLastError();
}

template <int D, bool KV>
hipError_t launch_rp(const BwdParams& P, int rp, int grid, hipStream_t s) {
  switch (rp) {
    case 0: return KV ? launch_dkdv_t<D, 0>(P, grid, s) : launch_dq_t<D, 0>(P, grid, s);
    case 16: return KV ? launch_dkdv_t<D, 16>(P, grid, s) : launch_dq_t<D, 16>(P, grid, s);
    case 32: return KV ? launch_dkdv_t<D, 32>(P, grid, s) : launch_dq_t<D, 32>(P, grid, s);
    case 48: return KV ? launch_dkdv_t<D, 48>(P, grid, s) : launch_dq_t<D, 48>(P, grid, s);
    case 64: return KV ? launch_dkdv_t<D, 64>(P, grid, s) : launch_dq_t<D, 64>(P, grid, s);
  }
  return hipErrorInvalidValue;
}

}  // namespace

hipError_t launch_bwd_delta(const BwdParams& P, hipStream_t s) {
  const Problem& p = P.p;
  const int64_t nrows = p.varlen ? (int64_t)p.total_q : (int64_t)p.nseq * p.sq;
  if (nrows > 0) {
    const int64_t threads = nrows * p.H * (p.D / 8);
    const int64_t grid = (threads + 255) / 256;
    if (p.D == 64)
      hipLaunchKernelGGL((delta_kernel<64>), dim3((unsigned)grid), dim3(256), 0, s, P, nrows);
    else
      hipLaunchKernelGGL((delta_kernel<128>), dim3((unsigned)grid), dim3(256), 0, s, P, nrows);
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

hipError_t launch_bwd_dkdv(const BwdParams& P, int rp, int grid, hipStream_t s) {
  if (grid <= 0) return hipSuccess;
  return P.p.D == 64 ? launch_rp<64, true>(P, rp, grid, s) : launch_rp<128, true>(P, rp, grid, s);
}

hipError_t launch_bwd_dq(const BwdParams& P, int rp, int grid, hipStream_t s) {
  if (grid <= 0) return hipSuccess;
  return P.p.D == 64 ? launch_rp<64, false>(P, rp, grid, s) : launch_rp<128, false>(P, rp, grid, s);
}

hipError_t launch_bwd_dgs(const BwdParams& P, int nparts, hipStream_t s) {
  if (P.p.H_G <= 0) return hipSuccess;
  hipLaunchKernelGGL(dgs_reduce_kernel, dim3(P.p.H_G), dim3(256), 0, s, P.dgs_partial,
                     nparts / P.p.H, P.p.H, P.dgs);
  return hipGetLastError();
}

}  // namespace fna2
