// fna2_bwd_dkdv.hip — dK, dV, dRk for gfx950.
//
// Replaces _fna2_bwd_dkdv_kernel / _fna2_bwd_dkdv_varlen_kernel
// (FNA2/flash_naylis_attn.py:390-553, :929-1076).
//
// One workgroup = 4 waves = 128 keys of one (sequence, KV head); wave w owns
// keys 32w..32w+31 and keeps K | Rk and V rows in registers (the B operands
// of S = Qa Ka^T and dP = dO V^T, one key per lane).  The workgroup walks
// the query heads of its GQA group and, for each, the 64-query blocks that
// can see its keys (causal: from the key tile's diagonal on).  Per block:
//   S, dP      (64 x 32 per wave)       A operands: Q | bf16(b Rq) and dO rows
//   P  = exp(S - LSE),  dS = P (dP - delta)
//   dV^T  += dO^T P                    A operand: dO^T by transpose reads
//   acc^T += [Q | Rq]^T dS             A operand: (Q | Rq)^T by transpose reads
// and the epilogue writes dK = a c acc_D, dRk = b c acc_R (b c = graph_scale).
// The rank part of the score operand is rounded as bf16(b Rq) from the raw
// Rq tile, as the forward does, and the sign/zero factor a of the augmented
// query rides on the stationary K (exact), so the recomputed S equals the
// forward's bit for bit.
// dK and dV accumulate over the whole GQA group in fp32 registers: no atomics.
// Q, Rq, dO, LSE and delta tiles stream in by DMA through a three-stage ring
// of separate LDS objects (the loop is unrolled by three so that the compiler
// can prove reads and in-flight DMA never alias).
#include "fna2_kernels.h"
#include "fna2_tile.h"

namespace fna2 {

namespace {

template <int D, int RPL>
struct KvCfg {
  static constexpr int NW = 4;
  static constexpr int BN = kKvBN;  // keys per workgroup
  static constexpr int BM = kKvBM;  // queries per step
  static constexpr int CD = D / 8;
  static constexpr int CR = RPL > 0 ? RPL / 8 : 4;
  static constexpr int KSD = D / 16;
  static constexpr int KSR = RPL / 16;
  static constexpr int NDB = D / 32;
  static constexpr int NRB = RPL / 32;
  static constexpr int QB = BM * D * 2;
  static constexpr int RB = BM * RPL * 2;
  static constexpr int OB = BM * D * 2;
  static constexpr int LB = 4 * BM * 4;  // LSE, delta, two scratch rows
  static constexpr int STAGE = QB + RB + OB + LB;
  // DMA instructions each wave issues per step (LSE/delta: one dword load).
  static constexpr int PER_STEP = 2 * Dma<BM, CD, NW>::PER_WAVE +
                                  (RPL > 0 ? Dma<BM, CR, NW>::PER_WAVE : 0) + 1;
};

template <int D, int RPL>
__device__ __forceinline__ void dkdv_body(const BwdParams& P) {
  using C = KvCfg<D, RPL>;
  __shared__ __attribute__((aligned(1024))) uint8_t st0[C::STAGE];
  __shared__ __attribute__((aligned(1024))) uint8_t st1[C::STAGE];
  __shared__ __attribute__((aligned(1024))) uint8_t st2[C::STAGE];
  const Problem& p = P.p;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = uni(tid >> 6);
  const int l32 = lane & 31, hl = lane >> 5;
  const int kvh = blockIdx.x % p.H_KV;
  const int tix = blockIdx.x / p.H_KV;
  int b, kt;
  if (P.tiles_k) {
    if (tix >= uni(*P.n_tiles_k)) return;
    const int2 t = P.tiles_k[tix];
    b = uni(t.x);
    kt = uni(t.y);
  } else {
    b = tix % p.nseq;
    kt = tix / p.nseq;
  }
  const SeqExt e = seq_ext_uniform(p, b);
  const int k0t = kt * C::BN;
  const int key = k0t + wv * 32 + l32;  // this lane's key
  const bool kvalid = key < e.lk;
  const int wk0 = k0t + wv * 32;
  const bool wave_keys = wk0 < e.lk;
  const int krows = max(min(C::BN, e.lk - k0t), 0);

  // Stationary K and V rows (B operands): lane holds row `key`, 8 features
  // 16s + 8hl .. +7 per step s.
  const uint16_t* kb = seq_base<const uint16_t>(P.k, p, b, e.k0, kvh);
  const uint16_t* vb = seq_base<const uint16_t>(P.v, p, b, e.k0, kvh);
  bf16x8 kreg[C::KSD + C::KSR];
  bf16x8 vreg[C::KSD];
  {
    const uint32_t krb = (uint32_t)P.k.ss * 2u, vrb = (uint32_t)P.v.ss * 2u;
    const auto rk = make_rsrc(kb + (int64_t)k0t * P.k.ss, (uint32_t)krows * krb);
    const auto rv = make_rsrc(vb + (int64_t)k0t * P.v.ss, (uint32_t)krows * vrb);
    const uint32_t ko = (uint32_t)(wv * 32 + l32) * krb + 16u * hl;
    const uint32_t vo = (uint32_t)(wv * 32 + l32) * vrb + 16u * hl;
    // The streamed Q tile is raw, so the factor a in {1, -1, 0} of the
    // augmented operand goes on K (exact): Q (a K) = (a Q) K.
    const uint32_t kxor = p.qa < 0.f ? 0x80008000u : 0u;
    const uint32_t kand = p.qa == 0.f ? 0u : 0xffffffffu;
#pragma unroll
    for (int s = 0; s < C::KSD; ++s) {
      u32x4 kv = __builtin_amdgcn_raw_buffer_load_b128(rk, ko + 32u * s, 0, 0);
#pragma unroll
      for (int i = 0; i < 4; ++i) kv[i] = (kv[i] & kand) ^ kxor;
      kreg[s] = as_bf16x8(kv);
      vreg[s] = as_bf16x8(__builtin_amdgcn_raw_buffer_load_b128(rv, vo + 32u * s, 0, 0));
    }
  }
  // Rank part of the stationary K operand for query head h (raw R_k).
  auto load_rk = [&](int h) {
    if constexpr (C::KSR > 0) {
      const bool graph = h < p.H_G;
      const uint32_t rrb = (uint32_t)P.rk.ss * 2u;
      const uint16_t* rkb = graph ? seq_base<const uint16_t>(P.rk, p, b, e.k0, h) : kb;
      const auto rr = make_rsrc(rkb + (int64_t)k0t * P.rk.ss, graph ? (uint32_t)krows * rrb : 0u);
      const uint32_t ro = (uint32_t)(wv * 32 + l32) * rrb + 16u * hl;
#pragma unroll
      for (int s = 0; s < C::KSR; ++s) {
        const bool in = (2 * s + hl) * 8 < p.R;
        kreg[C::KSD + s] =
            as_bf16x8(__builtin_amdgcn_raw_buffer_load_b128(rr, in ? ro + 32u * s : kOOB, 0, 0));
      }
    }
  };

  f32x16 dvacc[C::NDB];
  f32x16 dkacc[C::NDB + C::NRB];
#pragma unroll
  for (int i = 0; i < C::NDB; ++i) dvacc[i] = f32x16{};
#pragma unroll
  for (int i = 0; i < C::NDB + C::NRB; ++i) dkacc[i] = f32x16{};

  // Query blocks that can see this key tile; iterations walk (head, block).
  const int qb_lo = p.causal ? k0t / C::BM : 0;
  const int nqb = max(cdiv(e.lq, C::BM) - qb_lo, 0);
  const int total = p.group * nqb;

  // DMA plans for the streamed tiles.
  const uint32_t qrb = (uint32_t)P.q.ss * 2u, orb = (uint32_t)P.dout.ss * 2u;
  const uint32_t srb = (uint32_t)P.rq.ss * 2u;
  Dma<C::BM, C::CD, C::NW> dmq, dmo;
  Dma<C::BM, C::CR, C::NW> dmr;
  dmq.init(wv, lane, qrb, C::CD);
  dmo.init(wv, lane, orb, C::CD);
  if constexpr (RPL > 0) dmr.init(wv, lane, srb, p.R / 8);
  const uint32_t lrb = (uint32_t)P.lse.ss * 4u, drb = (uint32_t)P.delta.ss * 4u;
  const bool is_delta = (wv & 1) != 0;                 // waves 1, 3 load delta
  const int lslot = (wv & 1) * C::BM * 4 + (wv >> 1) * 2 * C::BM * 4;  // 2, 3: scratch rows
  const uint32_t loff = (uint32_t)lane * (is_delta ? drb : lrb);

  auto issue = [&](int it, uint8_t* st) {
    const int hi = it / nqb;
    const int qblk = qb_lo + (it - hi * nqb);
    const int h = kvh * p.group + hi;
    const int qbase = qblk * C::BM;
    const uint32_t rows = (uint32_t)max(min(C::BM, e.lq - qbase), 0);
    const uint16_t* qb = seq_base<const uint16_t>(P.q, p, b, e.q0, h);
    const uint16_t* ob = seq_base<const uint16_t>(P.dout, p, b, e.q0, h);
    dmq.issue(make_rsrc(qb + (int64_t)qbase * P.q.ss, rows * qrb), st, wv);
    if constexpr (RPL > 0) {
      const bool graph = h < p.H_G;
      const uint16_t* sb = graph ? seq_base<const uint16_t>(P.rq, p, b, e.q0, h) : qb;
      dmr.issue(make_rsrc(sb + (int64_t)qbase * P.rq.ss, graph ? rows * srb : 0u), st + C::QB,
                wv);
    }
    dmo.issue(make_rsrc(ob + (int64_t)qbase * P.dout.ss, rows * orb), st + C::QB + C::RB, wv);
    const float* lb = is_delta ? seq_base<const float>(P.delta, p, b, e.q0, h)
                               : seq_base<const float>(P.lse, p, b, e.q0, h);
    const int64_t lss = is_delta ? P.delta.ss : P.lse.ss;
    const auto rl = make_rsrc(lb + (int64_t)qbase * lss, rows * (is_delta ? drb : lrb));
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        rl, (lds_void*)(st + C::QB + C::RB + C::OB + lslot), 4, loff, 0, 0, 0);
  };

  // Per head: dRk, and this wave's d_gs partial
  //   sum_k <Rk_k, acc_R[k]> = sum_{q,k} dS_qk <Rq_q, Rk_k>  (the head's d_gs).
  // Lane half hl holds acc_R features 32f + 8g + 4hl + j and Rk features
  // 16s + 8hl + e (kreg[KSD + s]); for g % 2 == hl both are local, otherwise
  // the partner lane (lane ^ 32) holds the Rk values and sends them over.
  // Rows of keys past the sequence have Rk = 0 and contribute nothing.
  auto write_drk = [&](int h) {
    if constexpr (C::NRB > 0) {
      if (h >= p.H_G) return;
      float gp = 0.f;
#pragma unroll
      for (int f = 0; f < C::NRB; ++f) {
        const u32x4 r0 = as_u32x4(kreg[C::KSD + 2 * f]), r1 = as_u32x4(kreg[C::KSD + 2 * f + 1]);
        u32x2 sent[2], got[2];
        sent[0][0] = hl ? r0[0] : r0[2];
        sent[0][1] = hl ? r0[1] : r0[3];
        sent[1][0] = hl ? r1[0] : r1[2];
        sent[1][1] = hl ? r1[1] : r1[3];
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j) got[i][j] = __shfl_xor(sent[i][j], 32);
        const f32x16& a = dkacc[C::NDB + f];
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const u32x4& rr = (g >> 1) ? r1 : r0;
          const bool own = (g & 1) == hl;
          const uint32_t wa = own ? (hl ? rr[2] : rr[0]) : got[g >> 1][0];
          const uint32_t wb = own ? (hl ? rr[3] : rr[1]) : got[g >> 1][1];
          gp += bf16_lo(wa) * a[4 * g] + bf16_hi(wa) * a[4 * g + 1] + bf16_lo(wb) * a[4 * g + 2] +
                bf16_hi(wb) * a[4 * g + 3];
        }
      }
#pragma unroll
      for (int off = 32; off > 0; off >>= 1) gp += __shfl_xor(gp, off);
      if (lane == 0) P.dgs_partial[((int64_t)tix * 4 + wv) * p.H_G + h] = gp;
      if (kvalid) {
        const float sr = P.gs[h];  // dRk = b c acc_R with b c = graph_scale
        uint16_t* rrow = seq_base<uint16_t>(P.drk, p, b, e.k0, h) + (int64_t)key * P.drk.ss;
#pragma unroll
        for (int f = 0; f < C::NRB; ++f)
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const int rf = f * 32 + 8 * g + 4 * hl;
            if (rf < p.R) {
              const f32x16& a = dkacc[C::NDB + f];
              u32x2 val;
              val[0] = pack_bf16(sr * a[4 * g], sr * a[4 * g + 1]);
              val[1] = pack_bf16(sr * a[4 * g + 2], sr * a[4 * g + 3]);
              *(u32x2*)(rrow + rf) = val;
            }
          }
      }
    }
  };

  const TrLane tl(lane);

  // One query block: compute on `cur`; start the DMA for it + 2 into `nxt`.
  auto step = [&](int it, const uint8_t* cur, uint8_t* nxt) {
    if (it + 1 < total) ring_barrier<C::PER_STEP>(); else ring_barrier<0>();
    if (it + 2 < total) issue(it + 2, nxt);
    __builtin_amdgcn_sched_barrier(0);
    const int hi = it / nqb;
    const int qi = it - hi * nqb;
    const int h = kvh * p.group + hi;
    const bool graph = (RPL > 0) && (h < p.H_G);
    const float bh = graph ? P.gs[h] / p.c : 0.f;
    if (qi == 0 && it > 0) {  // next head of the GQA group
      load_rk(h);
#pragma unroll
      for (int i = C::NDB; i < C::NDB + C::NRB; ++i) dkacc[i] = f32x16{};
    }
    const int qbase = (qb_lo + qi) * C::BM;
    const bool active = wave_keys && (!p.causal || qbase + C::BM - 1 >= wk0);
    const bool diag = p.causal && wk0 + 31 > qbase;
    if (active) {
      const uint8_t* qt = cur;
      const uint8_t* rt = cur + C::QB;
      const uint8_t* ot = cur + C::QB + C::RB;
      const float* ls = (const float*)(cur + C::QB + C::RB + C::OB);
      const int nrs = graph ? cdiv(p.R, 16) : 0;
      bf16x8 pb[2][2], db[2][2];
#pragma unroll
      for (int rb = 0; rb < 2; ++rb) {
        const int row = rb * 32 + l32;
        f32x16 sacc = f32x16{}, dpacc = f32x16{};
#pragma unroll
        for (int s = 0; s < C::KSD; ++s) sacc = mfma32(row_read<C::CD>(qt, row, 2 * s + hl), kreg[s], sacc);
        if constexpr (C::KSR > 0) {
#pragma unroll
          for (int s = 0; s < C::KSR; ++s)
            if (s < nrs)
              sacc = mfma32(as_bf16x8(scale_bf16x8(as_u32x4(row_read<C::CR>(rt, row, 2 * s + hl)), bh)),
                            kreg[C::KSD + s], sacc);
        }
#pragma unroll
        for (int s = 0; s < C::KSD; ++s) dpacc = mfma32(row_read<C::CD>(ot, row, 2 * s + hl), vreg[s], dpacc);
        // P and dS for rows rb*32 + 8g + 4hl + j (accumulator register 4g + j).
        // Zero-filled query rows (past the sequence) have Q = dO = LSE =
        // delta = 0 and so P (dP - delta) = 0: only the causal diagonal needs
        // a mask; columns of keys past the sequence are never stored.
        if (diag) {
#pragma unroll
          for (int v = 0; v < 16; ++v) {
            const int q = qbase + rb * 32 + 8 * (v >> 2) + 4 * hl + (v & 3);
            sacc[v] = key <= q ? sacc[v] : kNegInf;
          }
        }
#pragma unroll
        for (int half = 0; half < 2; ++half) {
          u32x4 pk, dk;
#pragma unroll
          for (int g2 = 0; g2 < 2; ++g2) {
            const int g = 2 * half + g2;
            const int r0 = rb * 32 + 8 * g + 4 * hl;
            const f32x4_t lse4 = *(const f32x4_t*)(ls + r0);
            const f32x4_t dl4 = *(const f32x4_t*)(ls + C::BM + r0);
            float pv[4], dv[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              const int v = 4 * g + j;
              pv[j] = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[v], p.c2, -lse4[j] * kLog2e));
              dv[j] = pv[j] * (dpacc[v] - dl4[j]);
            }
            pk[2 * g2] = pack_bf16(pv[0], pv[1]);
            pk[2 * g2 + 1] = pack_bf16(pv[2], pv[3]);
            dk[2 * g2] = pack_bf16(dv[0], dv[1]);
            dk[2 * g2 + 1] = pack_bf16(dv[2], dv[3]);
          }
          pb[rb][half] = as_bf16x8(pk);
          db[rb][half] = as_bf16x8(dk);
        }
      }
      // dV^T += dO^T P ; dKa^T += Qa^T dA
#pragma unroll
      for (int rb = 0; rb < 2; ++rb)
#pragma unroll
        for (int half = 0; half < 2; ++half) {
          const int k0 = rb * 32 + 16 * half;
#pragma unroll
          for (int d = 0; d < C::NDB; ++d)
            dvacc[d] = mfma32(tr_operand<C::CD>(ot, tl, k0, 32 * d), pb[rb][half], dvacc[d]);
#pragma unroll
          for (int f = 0; f < C::NDB; ++f)
            dkacc[f] = mfma32(tr_operand<C::CD>(qt, tl, k0, 32 * f), db[rb][half], dkacc[f]);
          if constexpr (C::NRB > 0) {
            if (graph) {
#pragma unroll
              for (int f = 0; f < C::NRB; ++f)
                dkacc[C::NDB + f] =
                    mfma32(tr_operand<C::CR>(rt, tl, k0, 32 * f), db[rb][half], dkacc[C::NDB + f]);
            }
          }
        }
    }
    if (qi == nqb - 1) write_drk(h);  // last block of this head
  };

  load_rk(kvh * p.group);
  if (total > 0) issue(0, st0);
  if (total > 1) issue(1, st1);
  for (int it = 0; it < total; it += 3) {
    step(it, st0, st2);
    if (it + 1 < total) step(it + 1, st1, st0);
    if (it + 2 < total) step(it + 2, st2, st1);
  }
  if (total == 0) {
    // no query sees these keys: dRk of every graph head in the group is zero
    for (int hi = 0; hi < p.group; ++hi) write_drk(kvh * p.group + hi);
  }

  if (kvalid) {
    const float sk = p.qa * p.c;  // dK = a c acc_D
    uint16_t* krow = seq_base<uint16_t>(P.dk, p, b, e.k0, kvh) + (int64_t)key * P.dk.ss;
    uint16_t* vrow = seq_base<uint16_t>(P.dv, p, b, e.k0, kvh) + (int64_t)key * P.dv.ss;
#pragma unroll
    for (int d = 0; d < C::NDB; ++d)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int c0 = d * 32 + 8 * g + 4 * hl;
        u32x2 kv, vv;
        kv[0] = pack_bf16(sk * dkacc[d][4 * g], sk * dkacc[d][4 * g + 1]);
        kv[1] = pack_bf16(sk * dkacc[d][4 * g + 2], sk * dkacc[d][4 * g + 3]);
        vv[0] = pack_bf16(dvacc[d][4 * g], dvacc[d][4 * g + 1]);
        vv[1] = pack_bf16(dvacc[d][4 * g + 2], dvacc[d][4 * g + 3]);
        *(u32x2*)(krow + c0) = kv;
        *(u32x2*)(vrow + c0) = vv;
      }
  }
}

// One non-template kernel per (D, padded rank) so that each has a host stub.
#define FNA2_DKDV_KERNEL(D, RPL)                                                    \
  __global__ __launch_bounds__(256, 1) void dkdv_kernel_d##D##_r##RPL(const BwdParams P) { \
    dkdv_body<D, RPL>(P);                                                           \
  }
FNA2_DKDV_KERNEL(64, 0)
FNA2_DKDV_KERNEL(64, 32)
FNA2_DKDV_KERNEL(64, 64)
FNA2_DKDV_KERNEL(128, 0)
FNA2_DKDV_KERNEL(128, 32)
FNA2_DKDV_KERNEL(128, 64)
#undef FNA2_DKDV_KERNEL

}  // namespace

hipError_t launch_bwd_dkdv(const BwdParams& P, int rpl, int grid, hipStream_t s) {
  if (grid <= 0) return hipSuccess;
  void (*k)(const BwdParams) = nullptr;
  if (P.p.D == 64)
    k = rpl == 0 ? dkdv_kernel_d64_r0 : rpl == 32 ? dkdv_kernel_d64_r32 : dkdv_kernel_d64_r64;
  if (P.p.D == 128)
    k = rpl == 0 ? dkdv_kernel_d128_r0 : rpl == 32 ? dkdv_kernel_d128_r32 : dkdv_kernel_d128_r64;
  if (!k || (rpl != 0 && rpl != 32 && rpl != 64)) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k, dim3(grid), dim3(256), 0, s, P);
  return hipGetLastError();
}

}  // namespace fna2
