// fna2_bwd_dq.hip — dQ, dRq (and delta) for gfx950.
//
// Replaces _fna2_bwd_dq_kernel / _fna2_bwd_dq_varlen_kernel
// (FNA2/flash_naylis_attn.py:561-693, :1085-1208).
//
// One workgroup = 4 waves = 128 queries of one (sequence, head); wave w owns
// queries 32w..32w+31 with Qa = [a Q | Rq] and dO rows in registers.
// The prologue also forms delta = sum_d O dO for these queries (fp32); the
// epilogue stores it and -LSE log2(e) for the dK/dV kernel, which runs after
// this one.
// Per key step (keys stream in by DMA through a two-stage ring):
//   S^T, dP^T  (keys x 32 queries)      A operands: K | Rk and V rows (LDS)
//   dS^T = P^T (dP^T - delta)
//   acc^T += Ka^T dS^T                  A operand: (K | Rk)^T by transpose reads
// and the epilogue writes dQ = a c acc_D, dRq = b c acc_R and the wave's
// partial of d_gs = sum_i <Rq_i, (dS Rk)_i> (a fixed-order pass sums them).
#include "fna2_kernels.h"
#include "fna2_tile.h"

namespace fna2 {

namespace {

template <int D, int RPL>
struct DqCfg {
  static constexpr int NW = 4;
  static constexpr int BM = kDqBM;  // queries per workgroup
  // keys per step: 32 keeps d = 128 within 2 waves per SIMD and d = 64
  // (rank <= 32) within 3; rank 64 at d = 64 steps 64 keys.
  static constexpr int BN = (D == 128 || RPL <= 32) ? 32 : kDqBN;
  static constexpr int NKB = BN / 32;               // 32-key blocks per step
  static constexpr int CD = D / 8;
  static constexpr int CR = RPL > 0 ? RPL / 8 : 4;
  static constexpr int KSD = D / 16;
  static constexpr int KSR = RPL / 16;
  static constexpr int NDB = D / 32;
  static constexpr int NRB = RPL / 32;
  // d = 128: K / V operand reads in flight ahead of the S / dP MFMAs, and
  // K^T operands ahead of the dQ MFMAs (register budget: two waves per SIMD)
  static constexpr int kAhead = 2;
  static constexpr int kAhead2 = 2;
  static constexpr int KB = BN * D * 2;
  static constexpr int RB = BN * RPL * 2;
  static constexpr int VB = BN * D * 2;
  static constexpr int STAGE = KB + RB + VB;
};

// Gradient rows of tokens outside [cu[0], cu[N]) belong to no tile: with a
// plan (no list-building launch in the backward) the workgroups of the dQ
// grid that have no tile zero them, 16 bytes per store.  w of nw: this
// workgroup among them (the host launches one row of workgroups more than
// the tile list can fill, so there always are some).
__device__ void zero_uncovered_rows(const BwdParams& P, int w, int nw) {
  const Problem& p = P.p;
  const int cq0 = uni(*const_space(p.cu_q)), cqn = uni(*const_space(p.cu_q + p.nseq));
  const int ck0 = uni(*const_space(p.cu_k)), ckn = uni(*const_space(p.cu_k + p.nseq));
  if (cq0 <= 0 && cqn >= p.total_q && ck0 <= 0 && ckn >= p.total_k) return;
  const int rows = max(p.total_q, p.total_k);
  const u32x4 z = u32x4{0u, 0u, 0u, 0u};
  auto clear = [&](const TView& t, int heads, int feat, int64_t row) {
    for (int h = 0; h < heads; ++h) {
      uint16_t* r = (uint16_t*)t.ptr + row * t.ss + (int64_t)h * t.sh;
      for (int f = 0; f < feat; f += 8) st16(r + f, z);
    }
  };
  for (int64_t t = (int64_t)w * blockDim.x + threadIdx.x; t < rows;
       t += (int64_t)nw * blockDim.x) {
    if (t < p.total_q && (t < cq0 || t >= cqn)) {
      clear(P.dq, p.H, p.D, t);
      if (p.H_G > 0) clear(P.drq, p.H_G, p.R, t);
    }
    if (t < p.total_k && (t < ck0 || t >= ckn)) {
      clear(P.dk, p.H_KV, p.D, t);
      clear(P.dv, p.H_KV, p.D, t);
      if (p.H_G > 0) clear(P.drk, p.H_G, p.R, t);
    }
  }
}

template <int D, int RPL, bool F16>
__device__ __forceinline__ void dq_body(const BwdParams& P) {
  using C = DqCfg<D, RPL>;
  __shared__ __attribute__((aligned(1024))) uint8_t st0[C::STAGE];
  __shared__ __attribute__((aligned(1024))) uint8_t st1[C::STAGE];
  const Problem& p = P.p;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = uni(tid >> 6);
  const int l32 = lane & 31, hl = lane >> 5;
  const int h = blockIdx.x % p.H;
  const int tix = blockIdx.x / p.H;
  int b, qt;
  SeqExt e;
  int slot = tix;  // the tile's d_gs partial rows (list order in dense mode is fixed)
  if (P.tiles_q) {
    const int nt = min(uni(*const_space(P.n_tiles_q)), P.q_tiles);
    if (tix >= nt) {
      if (P.zero_uncovered) zero_uncovered_rows(P, (tix - nt) * p.H + h, (int)gridDim.x - nt * p.H);
      return;
    }
    tile_decode(P.tiles_q, tix, b, qt, e);
    slot = tile_slot(P.tiles_q, tix);
  } else {
    const int nqt = cdiv(p.sq, C::BM);
    b = tix % p.nseq;
    qt = nqt - 1 - tix / p.nseq;
    e = seq_ext_uniform(p, b);
  }
  const int kvh = h / p.group;
  const bool graph = (RPL > 0) && (h < p.H_G);
  const float bh = uni_f(graph ? *const_space(P.gs + h) / p.c : 0.f);
  const int nrs = graph ? cdiv(p.R, 16) : 0;
  // d = 128: the rank MFMAs run unconditionally (rank features past R and a
  // vanilla head's rank operands are zeros on both sides; a branch around
  // them made the compiler zero the accumulator registers before it: c4 dQ
  // -4.8%, c3 -1.2 us).  At d = 64 the branch measured faster (c2, c5).
  constexpr bool RANK_ALL = D == 128;

  const uint16_t* qb = seq_base<const uint16_t>(P.q, p, b, e.q0, h);
  const uint16_t* ob = seq_base<const uint16_t>(P.dout, p, b, e.q0, h);
  const uint16_t* kb = seq_base<const uint16_t>(P.k, p, b, e.k0, kvh);
  const uint16_t* vb = seq_base<const uint16_t>(P.v, p, b, e.k0, kvh);
  const uint16_t* rqb = graph ? seq_base<const uint16_t>(P.rq, p, b, e.q0, h) : qb;
  const uint16_t* rkb = graph ? seq_base<const uint16_t>(P.rk, p, b, e.k0, h) : kb;

  const int q0 = qt * C::BM;
  const int qrow = q0 + wv * 32 + l32;
  const bool qvalid = qrow < e.lq;
  const int wq0 = q0 + wv * 32;
  const int wq_last = min(wq0 + 31, e.lq - 1);
  const int qrows = max(min(C::BM, e.lq - q0), 0);

  int kv_hi = e.lk;
  if (p.causal) kv_hi = min(kv_hi, min(e.lq, q0 + C::BM));
  const int nkb = cdiv(max(kv_hi, 0), C::BN);

  const uint32_t krb = (uint32_t)P.k.ss * 2u, vrb = (uint32_t)P.v.ss * 2u;
  const uint32_t rkrb = (uint32_t)P.rk.ss * 2u;
  Dma<C::BN, C::CD, C::NW> dk, dv;
  Dma<C::BN, C::CR, C::NW> dr;
  dk.init(wv, lane, krb, C::CD);
  dv.init(wv, lane, vrb, C::CD);
  if constexpr (RPL > 0) dr.init(wv, lane, rkrb, p.R / 8);
  auto issue = [&](int it, uint8_t* st) {
    const int k0 = it * C::BN;
    const uint32_t rows = (uint32_t)max(min(C::BN, e.lk - k0), 0);
    dk.issue(make_rsrc(kb + (int64_t)k0 * P.k.ss, rows * krb), st, wv);
    if constexpr (RPL > 0) {
      // (RANK_ALL: a vanilla head's rank tile is a zero-size range, so the
      // DMA writes zeros and its rank MFMAs add exact zeros)
      if (RANK_ALL || graph)
        dr.issue(make_rsrc(rkb + (int64_t)k0 * P.rk.ss, graph ? rows * rkrb : 0u), st + C::KB, wv);
    }
    dv.issue(make_rsrc(vb + (int64_t)k0 * P.v.ss, rows * vrb), st + C::KB + C::RB, wv);
  };

  // The first key tile's DMA goes out before the row loads below, so the
  // two latencies overlap instead of adding up.
  if (nkb > 0) issue(0, st0);
  __builtin_amdgcn_sched_barrier(0);

  // Stationary B operands: Qa and dO rows of this lane's query.
  bf16x8 qreg[C::KSD + C::KSR];
  bf16x8 oreg[C::KSD];
  // d = 64: raw Rq in accumulator layout for the d_gs partial, loaded with
  // the rows (d = 128 derives it from the query registers at the end, as it
  // has no registers to spare).
  constexpr bool RQ_COPY = D == 64 && C::NRB > 0;
  u32x2 rq_epi[RQ_COPY ? C::NRB : 1][4];
  float lse2 = 0.f, dl = 0.f, lse_raw = 0.f;
  {
    const uint32_t rb = (uint32_t)P.q.ss * 2u, orb = (uint32_t)P.dout.ss * 2u;
    const auto rs = make_rsrc(qb + (int64_t)q0 * P.q.ss, (uint32_t)qrows * rb);
    const auto ro = make_rsrc(ob + (int64_t)q0 * P.dout.ss, (uint32_t)qrows * orb);
    const uint32_t vq = (uint32_t)(wv * 32 + l32) * rb + 16u * hl;
    const uint32_t vo = (uint32_t)(wv * 32 + l32) * orb + 16u * hl;
    const uint32_t qxor = p.qa < 0.f ? 0x80008000u : 0u;
    const uint32_t qand = p.qa == 0.f ? 0u : 0xffffffffu;
    {
      const uint32_t lrb = (uint32_t)P.lse.ss * 4u;
      const auto rl = make_rsrc(seq_base<const float>(P.lse, p, b, e.q0, h) + (int64_t)q0 * P.lse.ss,
                                (uint32_t)qrows * lrb);
      lse_raw = __builtin_bit_cast(
          float, __builtin_amdgcn_raw_buffer_load_b32(rl, (uint32_t)(wv * 32 + l32) * lrb, 0, 0));
    }
#pragma unroll
    for (int s = 0; s < C::KSD; ++s) {
      u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rs, vq + 32u * s, 0, 0);
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = (v[i] & qand) ^ qxor;
      qreg[s] = as_bf16x8(v);
      oreg[s] = as_bf16x8(__builtin_amdgcn_raw_buffer_load_b128(ro, vo + 32u * s, 0, 0));
    }
    if constexpr (C::KSR > 0) {
      const uint32_t rrb = (uint32_t)P.rq.ss * 2u;
      const auto rr = make_rsrc(rqb + (int64_t)q0 * P.rq.ss, graph ? (uint32_t)qrows * rrb : 0u);
      const uint32_t vr = (uint32_t)(wv * 32 + l32) * rrb + 16u * hl;
#pragma unroll
      for (int s = 0; s < C::KSR; ++s) {
        const bool in = (2 * s + hl) * 8 < p.R;
        qreg[C::KSD + s] =
            as_bf16x8(__builtin_amdgcn_raw_buffer_load_b128(rr, in ? vr + 32u * s : kOOB, 0, 0));
      }
      if constexpr (RQ_COPY) {
#pragma unroll
        for (int f = 0; f < C::NRB; ++f)
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const int rf = f * 32 + 8 * g + 4 * hl;
            rq_epi[f][g] = __builtin_amdgcn_raw_buffer_load_b64(
                rr, rf < p.R ? (uint32_t)(wv * 32 + l32) * rrb + 2u * rf : kOOB, 0, 0);
          }
      }
    }
    // delta = sum_d O dO for this lane's query: the lane pair (hl = 0, 1)
    // holds the row's dO chunks, so O is read in the same layout.
    {
      const uint32_t yrb = (uint32_t)P.o.ss * 2u;
      const uint16_t* yb = seq_base<const uint16_t>(P.o, p, b, e.q0, h);
      const auto ry = make_rsrc(yb + (int64_t)q0 * P.o.ss, (uint32_t)qrows * yrb);
      const uint32_t vy = (uint32_t)(wv * 32 + l32) * yrb + 16u * hl;
#pragma unroll
      for (int s = 0; s < C::KSD; ++s) {
        const u32x4 y = __builtin_amdgcn_raw_buffer_load_b128(ry, vy + 32u * s, 0, 0);
        const u32x4 o = as_u32x4(oreg[s]);
#pragma unroll
        for (int i = 0; i < 4; ++i)
          dl += elt_lo<F16>(y[i]) * elt_lo<F16>(o[i]) + elt_hi<F16>(y[i]) * elt_hi<F16>(o[i]);
      }
      dl += __shfl_xor(dl, 32);
    }
    lse2 = lse_raw * kLog2e;
  }

  f32x16 acc[C::NDB + C::NRB];
#pragma unroll
  for (int i = 0; i < C::NDB + C::NRB; ++i) acc[i] = f32x16{};
  const TrLane tl(lane);
  const RowLane rdl(lane);

  auto step = [&](int it, const uint8_t* cur, uint8_t* nxt) {
    ring_barrier<0>();
    if (it + 1 < nkb) issue(it + 1, nxt);
    __builtin_amdgcn_sched_barrier(0);
    const int kbase = it * C::BN;
    const bool active = (wq0 <= wq_last) && (!p.causal || kbase <= wq_last);
    if (!active) return;
    const bool diag = p.causal && kbase + C::BN - 1 > wq0;
    const uint8_t* kt = cur;
    const uint8_t* rt = cur + C::KB;
    const uint8_t* vt = cur + C::KB + C::RB;
    // dS^T as B operands: in the element type for the dQ chain (K^T is of
    // that type) and in bf16 for the dRq chain (Rk^T is bf16); one array
    // when the two types agree.
    constexpr bool DBR = F16 && C::NRB > 0;
    bf16x8 db[C::NKB][2];
    bf16x8 dbr[DBR ? C::NKB : 1][2];
#pragma unroll
    for (int kb2 = 0; kb2 < C::NKB; ++kb2) {
      f32x16 sacc = f32x16{}, dpacc = f32x16{};
      // At d = 128 the S and dP chains run interleaved, their K and V
      // operand reads kAhead k-steps ahead of the MFMAs, issued before the
      // rank chain with (rank tile 32) that chain's Rk reads (read whether
      // or not the head has a rank part; unused then).  The scheduling
      // fences keep every read where it is issued, else the compiler, short
      // of registers, reads each operand just before its MFMA and waits for
      // it: c3 dQ 128.4 -> 123.3 us, c4 -4%.
      constexpr bool PIPE = D == 128;
      constexpr int A = PIPE ? C::kAhead : 1;
      bf16x8 kr[A], vr[A];
      constexpr bool RPRE = PIPE && C::KSR > 0 && C::KSR <= 2;
      bf16x8 rr[RPRE ? C::KSR : 1];
      if constexpr (PIPE) {
        if constexpr (RPRE) {
#pragma unroll
          for (int s = 0; s < C::KSR; ++s) rr[s] = row_read<C::BN>(rt, rdl, kb2 * 32, s);
        }
#pragma unroll
        for (int s = 0; s < A; ++s) {
          kr[s] = row_read<C::BN>(kt, rdl, kb2 * 32, s);
          vr[s] = row_read<C::BN>(vt, rdl, kb2 * 32, s);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      // S^T / c = b Rk Rq^T + K (a Q)^T: the rank chain, scaled by b in
      // fp32, then the head-dim chain on top.
      if constexpr (C::KSR > 0) {
#pragma unroll
        for (int s = 0; s < C::KSR; ++s)
          if (RANK_ALL || s < nrs)
            sacc = mfma32(RPRE ? rr[RPRE ? s : 0] : row_read<C::BN>(rt, rdl, kb2 * 32, s),
                          qreg[C::KSD + s], sacc);
        sacc *= bh;
      }
      if constexpr (PIPE) {
#pragma unroll
        for (int s = 0; s < C::KSD; ++s) {
          sacc = mfma_e<F16>(kr[s % A], qreg[s], sacc);
          dpacc = mfma_e<F16>(vr[s % A], oreg[s], dpacc);
          if (s + A < C::KSD) {
            kr[s % A] = row_read<C::BN>(kt, rdl, kb2 * 32, s + A);
            vr[s % A] = row_read<C::BN>(vt, rdl, kb2 * 32, s + A);
          }
          __builtin_amdgcn_sched_barrier(0);
        }
      } else {
#pragma unroll
        for (int s = 0; s < C::KSD; ++s)
          sacc = mfma_e<F16>(row_read<C::BN>(kt, rdl, kb2 * 32, s), qreg[s], sacc);
#pragma unroll
        for (int s = 0; s < C::KSD; ++s)
          dpacc = mfma_e<F16>(row_read<C::BN>(vt, rdl, kb2 * 32, s), oreg[s], dpacc);
      }
      // dS^T = P^T (dP^T - delta).  Zero-filled key rows (past the
      // sequence) and query rows give K = Rk = 0 or dO = 0 and contribute
      // nothing, so only the causal diagonal needs a mask.
      if (diag) {
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int key = kbase + kb2 * 32 + 8 * (v >> 2) + 4 * hl + (v & 3);
          sacc[v] = key <= qrow ? sacc[v] : kNegInf;
        }
      }
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        u32x4 dk4, dr4;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float dv2[2];
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            const int v = 8 * half + 2 * i + j;
            const float pr = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[v], p.c2, -lse2));
            dv2[j] = pr * (dpacc[v] - dl);
          }
          dk4[i] = pack_e<F16>(dv2[0], dv2[1]);
          if constexpr (DBR) dr4[i] = pack_bf16(dv2[0], dv2[1]);
        }
        db[kb2][half] = as_bf16x8(dk4);
        if constexpr (DBR) dbr[kb2][half] = as_bf16x8(dr4);
      }
    }
    // dQa^T += Ka^T dA^T (at d = 128 the head-dim part first, its operand
    // reads kAhead2 MFMAs ahead, then the rank part, whose Rk^T operands
    // (rank tile 32) are read with the first ones)
    constexpr bool RPRE2 = C::NKB == 1 && D == 128 && C::NRB == 1;
    bf16x8 rr2[2];
    if constexpr (C::NKB == 1 && D == 128) {
      constexpr int A = C::kAhead2, N = 2 * C::NDB;
      bf16x8 kr[A];
      if constexpr (RPRE2) {
        rr2[0] = tr_operand<C::BN>(rt, tl, 0, 0);
        rr2[1] = tr_operand<C::BN>(rt, tl, 16, 0);
      }
#pragma unroll
      for (int i = 0; i < A; ++i) kr[i] = tr_operand<C::BN>(kt, tl, 16 * (i / C::NDB), 32 * (i % C::NDB));
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < N; ++i) {
        const int half = i / C::NDB, f = i % C::NDB;
        acc[f] = mfma_e<F16>(kr[i % A], db[0][half], acc[f]);
        if (i + A < N)
          kr[i % A] = tr_operand<C::BN>(kt, tl, 16 * ((i + A) / C::NDB), 32 * ((i + A) % C::NDB));
        __builtin_amdgcn_sched_barrier(0);
      }
    }
#pragma unroll
    for (int kb2 = 0; kb2 < C::NKB; ++kb2)
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        const int k0 = kb2 * 32 + 16 * half;
        if constexpr (!(C::NKB == 1 && D == 128)) {
#pragma unroll
          for (int f = 0; f < C::NDB; ++f)
            acc[f] = mfma_e<F16>(tr_operand<C::BN>(kt, tl, k0, 32 * f), db[kb2][half], acc[f]);
        }
        if constexpr (C::NRB > 0) {
          if (graph) {
#pragma unroll
            for (int f = 0; f < C::NRB; ++f)
              acc[C::NDB + f] = mfma32(RPRE2 ? rr2[half] : tr_operand<C::BN>(rt, tl, k0, 32 * f),
                                       DBR ? dbr[DBR ? kb2 : 0][half] : db[kb2][half],
                                       acc[C::NDB + f]);
          }
        }
      }
  };

  for (int it = 0; it < nkb; it += 2) {
    step(it, st0, st1);
    if (it + 1 < nkb) step(it + 1, st1, st0);
  }

  // The loop accumulated dS = P (dP - delta); dA = c dS.  This lane's part
  // of the d_gs partial: <Rq_i, (dS Rk)_i> of its query row.
  // The accumulator holds rank features f*32 + 8g + 4hl + e of this lane's
  // row (e = 0..3).  At d = 128 they come from the query registers, which
  // hold features 16s + 8hl .. +7: half of the needed Rq values sit in the
  // partner lane (lane ^ 32), so each lane passes over the two dwords of
  // every rank k-step that the partner needs.
  float gpart = 0.f;
  if constexpr (C::NRB > 0) {
#pragma unroll
    for (int f = 0; f < C::NRB; ++f) {
      u32x2 rv[4];
      if constexpr (RQ_COPY) {
#pragma unroll
        for (int g = 0; g < 4; ++g) rv[g] = rq_epi[f][g];
      } else {
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          const u32x4 q = as_u32x4(qreg[C::KSD + 2 * f + t]);
          const uint32_t x0 = __shfl_xor(hl ? q[0] : q[2], 32);
          const uint32_t x1 = __shfl_xor(hl ? q[1] : q[3], 32);
          // this lane's half of features 32f + 16t + 8hl .. +7 that it
          // keeps (lower for hl = 0, upper for hl = 1), and the partner's
          const u32x2 own = hl ? u32x2{q[2], q[3]} : u32x2{q[0], q[1]};
          const u32x2 got = u32x2{x0, x1};
          rv[2 * t] = hl ? got : own;      // g = 2t:     features 16t + 4hl .. +3
          rv[2 * t + 1] = hl ? own : got;  // g = 2t + 1: features 16t + 8 + 4hl .. +3
        }
      }
      if (graph && qvalid) {
        const f32x16& a = acc[C::NDB + f];
#pragma unroll
        for (int g = 0; g < 4; ++g)
          if (f * 32 + 8 * g + 4 * hl < p.R)
            gpart += bf16_lo(rv[g][0]) * a[4 * g] + bf16_hi(rv[g][0]) * a[4 * g + 1] +
                     bf16_lo(rv[g][1]) * a[4 * g + 2] + bf16_hi(rv[g][1]) * a[4 * g + 3];
      }
    }
  }
  // Epilogue: the ring is idle once every wave has left the loop, so each
  // wave stages its 32 rows of dQ (then of dRq) there (wave w: stage w / 2,
  // half w % 2) and stores them as whole rows, 16 bytes per lane.
  using QS = RowStage<D>;
  static_assert(2 * QS::BYTES <= C::STAGE, "the epilogue staging fits in a ring stage");
  __syncthreads();
  uint8_t* obuf = (wv < 2 ? st0 : st1) + (wv & 1) * QS::BYTES;
  const int nrows = max(min(32, e.lq - wq0), 0);
  const float sq = p.qa * p.c;
#pragma unroll
  for (int d = 0; d < C::NDB; ++d)
#pragma unroll
    for (int g = 0; g < 4; ++g)
      QS::template put4<F16>(obuf, l32, d * 32 + 8 * g + 4 * hl, sq * acc[d][4 * g],
                             sq * acc[d][4 * g + 1], sq * acc[d][4 * g + 2],
                             sq * acc[d][4 * g + 3]);
  QS::store(obuf, seq_base<uint16_t>(P.dq, p, b, e.q0, h) + (int64_t)wq0 * P.dq.ss, P.dq.ss,
            nrows, QS::CPR, lane);
  if constexpr (C::NRB > 0) {
    if (graph) {
      using RS = RowStage<RPL>;
      static_assert(RS::BYTES <= QS::BYTES, "dRq rows fit where the dQ rows were");
      const float sr = bh * p.c;
#pragma unroll
      for (int f = 0; f < C::NRB; ++f)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int rf = f * 32 + 8 * g + 4 * hl;
          const f32x16& a = acc[C::NDB + f];
          if (rf < p.R)
            RS::put4(obuf, l32, rf, sr * a[4 * g], sr * a[4 * g + 1], sr * a[4 * g + 2],
                     sr * a[4 * g + 3]);
        }
      RS::store(obuf, seq_base<uint16_t>(P.drq, p, b, e.q0, h) + (int64_t)wq0 * P.drq.ss,
                P.drq.ss, nrows, p.R / 8, lane);
    }
  }
  // For the dK/dV kernel: delta and -LSE log2(e).  They are stored here
  // rather than in the prologue, where the first ring barrier (vmcnt(0))
  // would wait for the writes to complete.
  if (qvalid && hl == 0) {
    seq_base<float>(P.delta, p, b, e.q0, h)[(int64_t)qrow * P.delta.ss] = dl;
    seq_base<float>(P.nlse, p, b, e.q0, h)[(int64_t)qrow * P.nlse.ss] = -lse2;
  }
  // d_gs partial of this wave: sum_i <Rq_i, (dS Rk)_i> over its queries.
  if constexpr (C::NRB > 0) {
    if (graph) {
#pragma unroll
      for (int off = 32; off > 0; off >>= 1) gpart += __shfl_xor(gpart, off);
      if (lane == 0 && slot < P.q_tiles) P.dgs_partial[((int64_t)slot * 4 + wv) * p.H_G + h] = gpart;
    }
  }
}

// WAVES: waves per SIMD the register budget is cut for.
#define FNA2_DQ_KERNEL(D, RPL, WAVES)                                                    \
  __global__ __launch_bounds__(256, WAVES) void dq_kernel_d##D##_r##RPL(const BwdParams P) { \
    dq_body<D, RPL, false>(P);                                                           \
  }                                                                                      \
  __global__ __launch_bounds__(256, WAVES) void dq_kernel_d##D##_r##RPL##_f16(             \
      const BwdParams P) {                                                               \
    dq_body<D, RPL, true>(P);                                                            \
  }
FNA2_DQ_KERNEL(64, 0, 3)
FNA2_DQ_KERNEL(64, 32, 3)
FNA2_DQ_KERNEL(64, 64, 2)
FNA2_DQ_KERNEL(128, 0, 2)
FNA2_DQ_KERNEL(128, 32, 2)
FNA2_DQ_KERNEL(128, 64, 2)
#undef FNA2_DQ_KERNEL

}  // namespace

hipError_t launch_bwd_dq(const BwdParams& P, int rpl, int grid, hipStream_t s) {
  if (grid <= 0) return hipSuccess;
  void (*k)(const BwdParams) = nullptr;
  if (P.p.f16) {
    if (P.p.D == 64)
      k = rpl == 0 ? dq_kernel_d64_r0_f16 : rpl == 32 ? dq_kernel_d64_r32_f16 : dq_kernel_d64_r64_f16;
    if (P.p.D == 128)
      k = rpl == 0 ? dq_kernel_d128_r0_f16 : rpl == 32 ? dq_kernel_d128_r32_f16 : dq_kernel_d128_r64_f16;
  } else {
    if (P.p.D == 64) k = rpl == 0 ? dq_kernel_d64_r0 : rpl == 32 ? dq_kernel_d64_r32 : dq_kernel_d64_r64;
    if (P.p.D == 128)
      k = rpl == 0 ? dq_kernel_d128_r0 : rpl == 32 ? dq_kernel_d128_r32 : dq_kernel_d128_r64;
  }
  if (!k || (rpl != 0 && rpl != 32 && rpl != 64)) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k, dim3(grid), dim3(256), 0, s, P);
  return hipGetLastError();
}

}  // namespace fna2
