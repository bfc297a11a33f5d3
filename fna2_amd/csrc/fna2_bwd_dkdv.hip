// fna2_bwd_dkdv.hip — dK, dV, dRk for gfx950.
//
// Replaces _fna2_bwd_dkdv_kernel / _fna2_bwd_dkdv_varlen_kernel
// (FNA2/flash_naylis_attn.py:390-553, :929-1076).
//
// Persistent: one workgroup per CU walks a list of work items, an item being
// the 128 keys of one key tile of one KV head; workgroup g takes items
// g, 2G-1-g, 2G+g, ... (snake order over a longest-first list).  Wave w owns
// keys 32w..32w+31 of the item and keeps K | Rk and V rows in registers (the
// B operands of S = Qa Ka^T and dP = dO V^T, one key per lane).  For each
// query head of the GQA group the item walks the 64-query blocks that can
// see its keys (causal: from the key tile's diagonal on).  Per block:
//   S, dP      (64 x 32 per wave)       A operands: Q | bf16(b Rq) and dO rows
//   P  = exp(S - LSE),  dS = P (dP - delta)
//   dV^T  += dO^T P                    A operand: dO^T by transpose reads
//   acc^T += [Q | bf16(b Rq)]^T dS     A operand: the same tiles transposed
// and the epilogue writes dK = a c acc_D, dRk = c acc_R (acc_R built from the
// rank operand bf16(b Rq), so c acc_R = graph_scale dS^T Rq).  The dQ kernel
// stores that operand, rounded exactly as the forward rounds it, with delta
// and -LSE log2(e); the sign/zero factor a of the augmented query rides on the
// stationary K (exact), so the recomputed S equals the forward's bit for bit.  dK and dV
// accumulate over the whole GQA group in fp32 registers: no atomics.
//
// Q, bf16(b Rq), dO, -LSE log2(e) and delta tiles stream in by DMA through a three-stage ring
// that runs two blocks ahead of the compute across item boundaries, so the
// next item's first tiles are in flight while the current item finishes.  At
// an item's last block, once its MFMAs are issued, the epilogue stores go out
// and the next item's K | Rk, V rows are loaded into the stationary
// registers.  The stages are separate LDS objects and the loop is unrolled by
// three so that the compiler can prove reads and in-flight DMA never alias.
#include "fna2_kernels.h"
#include "fna2_tile.h"

namespace fna2 {

namespace {

template <int D, int RPL>
struct KvCfg {
  static constexpr int NW = 4;
  static constexpr int BN = kKvBN;  // keys per item
  static constexpr int BM = kKvBM;  // queries per block
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
  static constexpr int ERS = D * 2 + 16;  // epilogue staging row stride (bytes)
  // DMA instructions each wave issues per block (LSE/delta: one dword load).
  static constexpr int PER_STEP = 2 * Dma<BM, CD, NW>::PER_WAVE +
                                  (RPL > 0 ? Dma<BM, CR, NW>::PER_WAVE : 0) + 1;
};

struct KvItem {
  int tix, b, kvh, k0t;  // key tile index, sequence, KV head, first key
  SeqExt e;
  int qb_lo, nqb;        // first query block that sees the tile; blocks per head
};

// Position in a workgroup's program: item (round r), head hi, block qi.
struct KvCursor {
  int r, hi, qi;
  bool done;
  KvItem it;
};

template <int D, int RPL>
__device__ __forceinline__ void dkdv_body(const BwdParams& P) {
  using C = KvCfg<D, RPL>;
  __shared__ __attribute__((aligned(1024))) uint8_t st0[C::STAGE];
  __shared__ __attribute__((aligned(1024))) uint8_t st1[C::STAGE];
  __shared__ __attribute__((aligned(1024))) uint8_t st2[C::STAGE];
  __shared__ __attribute__((aligned(16))) uint8_t epi[C::NW * 32 * C::ERS];
  const Problem& p = P.p;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = uni(tid >> 6);
  const int l32 = lane & 31, hl = lane >> 5;
  const int krow = wv * 32 + l32;  // this lane's key within the item
  const int G = gridDim.x, g = blockIdx.x;
  const int n_items =
      (P.tiles_k ? uni(*P.n_tiles_k) : p.nseq * cdiv(p.sk, C::BN)) * p.H_KV;

  auto decode = [&](int w) {
    KvItem x;
    x.tix = w / p.H_KV;
    x.kvh = w - x.tix * p.H_KV;
    int kt;
    if (P.tiles_k) {
      tile_decode(P.tiles_k, x.tix, x.b, kt, x.e);
    } else {
      x.b = x.tix % p.nseq;
      kt = x.tix / p.nseq;
      x.e = seq_ext_uniform(p, x.b);
    }
    x.k0t = kt * C::BN;
    x.qb_lo = p.causal ? x.k0t / C::BM : 0;
    x.nqb = max(cdiv(x.e.lq, C::BM) - x.qb_lo, 0);
    return x;
  };

  f32x16 dvacc[C::NDB];
  f32x16 dkacc[C::NDB + C::NRB];
  bf16x8 kreg[C::KSD + C::KSR];
  bf16x8 vreg[C::KSD];

  // Stationary rows of item x (B operands): lane holds key row krow,
  // features 16s + 8hl .. +7 for step s.  The streamed Q tile is raw, so the
  // factor a in {1, -1, 0} of the augmented operand goes on K (exact).
  const uint32_t kxor = p.qa < 0.f ? 0x80008000u : 0u;
  const uint32_t kand = p.qa == 0.f ? 0u : 0xffffffffu;
  auto load_kv = [&](const KvItem& x) {
    const uint32_t krows = (uint32_t)max(min(C::BN, x.e.lk - x.k0t), 0);
    const uint32_t krb = (uint32_t)P.k.ss * 2u, vrb = (uint32_t)P.v.ss * 2u;
    const uint16_t* kb = seq_base<const uint16_t>(P.k, p, x.b, x.e.k0, x.kvh);
    const uint16_t* vb = seq_base<const uint16_t>(P.v, p, x.b, x.e.k0, x.kvh);
    const auto rk = make_rsrc(kb + (int64_t)x.k0t * P.k.ss, krows * krb);
    const auto rv = make_rsrc(vb + (int64_t)x.k0t * P.v.ss, krows * vrb);
    const uint32_t ko = (uint32_t)krow * krb + 16u * hl;
    const uint32_t vo = (uint32_t)krow * vrb + 16u * hl;
#pragma unroll
    for (int s = 0; s < C::KSD; ++s) {
      kreg[s] = as_bf16x8(__builtin_amdgcn_raw_buffer_load_b128(rk, ko + 32u * s, 0, 0));
      vreg[s] = as_bf16x8(__builtin_amdgcn_raw_buffer_load_b128(rv, vo + 32u * s, 0, 0));
    }
    // (a = 1, the usual case, needs no transform, so nothing here waits for
    // the loads.)
    if (p.qa != 1.f) {
#pragma unroll
      for (int s = 0; s < C::KSD; ++s) {
        u32x4 kv = as_u32x4(kreg[s]);
#pragma unroll
        for (int i = 0; i < 4; ++i) kv[i] = (kv[i] & kand) ^ kxor;
        kreg[s] = as_bf16x8(kv);
      }
    }
  };
  // Rank part of the stationary K operand for query head h (raw Rk).
  auto load_rk = [&](const KvItem& x, int h) {
    if constexpr (C::KSR > 0) {
      const bool graph = h < p.H_G;
      const uint32_t krows = (uint32_t)max(min(C::BN, x.e.lk - x.k0t), 0);
      const uint32_t rrb = (uint32_t)P.rk.ss * 2u;
      const uint16_t* rkb = graph ? seq_base<const uint16_t>(P.rk, p, x.b, x.e.k0, h)
                                  : (const uint16_t*)P.rk.ptr;
      const auto rr = make_rsrc(rkb + (int64_t)x.k0t * P.rk.ss, graph ? krows * rrb : 0u);
      const uint32_t ro = (uint32_t)krow * rrb + 16u * hl;
#pragma unroll
      for (int s = 0; s < C::KSR; ++s) {
        const bool in = (2 * s + hl) * 8 < p.R;
        kreg[C::KSD + s] =
            as_bf16x8(__builtin_amdgcn_raw_buffer_load_b128(rr, in ? ro + 32u * s : kOOB, 0, 0));
      }
    }
  };

  // Per head: dRk = c acc_R (acc_R = dS^T bf16(b Rq) and b c = graph_scale).
  // zero: an item no query block sees.
  auto write_drk = [&](const KvItem& x, int h, bool zero) {
    if constexpr (C::NRB > 0) {
      const int key = x.k0t + krow;
      if (h < p.H_G && key < x.e.lk) {
        const float sr = zero ? 0.f : p.c;
        uint16_t* rrow = seq_base<uint16_t>(P.drk, p, x.b, x.e.k0, h) + (int64_t)key * P.drk.ss;
#pragma unroll
        for (int f = 0; f < C::NRB; ++f)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int rf = f * 32 + 8 * q + 4 * hl;
            if (rf < p.R) {
              const f32x16& a = dkacc[C::NDB + f];
              u32x2 val;
              val[0] = zero ? 0u : pack_bf16(sr * a[4 * q], sr * a[4 * q + 1]);
              val[1] = zero ? 0u : pack_bf16(sr * a[4 * q + 2], sr * a[4 * q + 3]);
              *(u32x2*)(rrow + rf) = val;
            }
          }
      }
    }
  };
  // dK = a c acc_D and dV: each wave stages its 32 rows through its own LDS
  // buffer so that a store instruction writes whole rows (4 rows of 16-byte
  // chunks for d = 128), instead of 64 scattered 8-byte pieces.
  uint8_t* obuf = epi + wv * 32 * C::ERS;
  auto write_rows = [&](const KvItem& x, const f32x16* acc, float sc, bool zero,
                        const TView& out) {
#pragma unroll
    for (int d = 0; d < C::NDB; ++d)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        u32x2 val;
        val[0] = zero ? 0u : pack_bf16(sc * acc[d][4 * q], sc * acc[d][4 * q + 1]);
        val[1] = zero ? 0u : pack_bf16(sc * acc[d][4 * q + 2], sc * acc[d][4 * q + 3]);
        *(u32x2*)(obuf + l32 * C::ERS + (d * 32 + 8 * q + 4 * hl) * 2) = val;
      }
    constexpr int CPR = D / 8;       // 16-byte chunks per row
    constexpr int RPI = 64 / CPR;    // rows per store instruction
    uint16_t* base = seq_base<uint16_t>(out, p, x.b, x.e.k0, x.kvh);
#pragma unroll
    for (int i = 0; i < 32 / RPI; ++i) {
      const int r = i * RPI + lane / CPR, ch = lane % CPR;
      const u32x4 v = *(const u32x4*)(obuf + r * C::ERS + ch * 16);
      const int key = x.k0t + wv * 32 + r;
      if (key < x.e.lk) st16(base + (int64_t)key * out.ss + ch * 8, v);
    }
  };
  auto write_dkdv = [&](const KvItem& x, bool zero) {
    write_rows(x, dkacc, p.qa * p.c, zero, P.dk);
    write_rows(x, dvacc, 1.f, zero, P.dv);
  };

  // ---- the program: items in snake order, then heads, then blocks ----
  // An item no query block can see (keys past every query under the causal
  // mask, or an empty query range) has zero gradients; the compute cursor
  // writes them as it passes.
  auto next_item = [&](KvCursor& c, bool compute) {
    for (;;) {
      ++c.r;
      const int w = c.r * G + ((c.r & 1) ? G - 1 - g : g);
      if (w >= n_items) {
        c.done = true;
        return;
      }
      c.it = decode(w);
      c.hi = 0;
      c.qi = 0;
      if (c.it.nqb > 0) return;
      if (compute) {
        write_dkdv(c.it, true);
        for (int hi = 0; hi < p.group; ++hi) write_drk(c.it, c.it.kvh * p.group + hi, true);
      }
    }
  };
  auto advance = [&](KvCursor& c, bool compute) {
    if (++c.qi < c.it.nqb) return;
    c.qi = 0;
    if (++c.hi < p.group) return;
    next_item(c, compute);
  };

  // DMA plans for the streamed tiles.
  const uint32_t qrb = (uint32_t)P.q.ss * 2u, orb = (uint32_t)P.dout.ss * 2u;
  const uint32_t srb = (uint32_t)P.rqs.ss * 2u;
  Dma<C::BM, C::CD, C::NW> dmq, dmo;
  Dma<C::BM, C::CR, C::NW> dmr;
  dmq.init(wv, lane, qrb, C::CD);
  dmo.init(wv, lane, orb, C::CD);
  if constexpr (RPL > 0) dmr.init(wv, lane, srb, C::CR);
  const uint32_t lrb = (uint32_t)P.nlse.ss * 4u, drb = (uint32_t)P.delta.ss * 4u;
  const bool is_delta = (wv & 1) != 0;                                 // waves 1, 3: delta
  const int lslot = (wv & 1) * C::BM * 4 + (wv >> 1) * 2 * C::BM * 4;  // 2, 3: scratch rows
  const uint32_t loff = (uint32_t)lane * (is_delta ? drb : lrb);

  auto issue = [&](const KvCursor& c, uint8_t* st) {
    const KvItem& x = c.it;
    const int h = x.kvh * p.group + c.hi;
    const int qbase = (x.qb_lo + c.qi) * C::BM;
    const uint32_t rows = (uint32_t)max(min(C::BM, x.e.lq - qbase), 0);
    const uint16_t* qb = seq_base<const uint16_t>(P.q, p, x.b, x.e.q0, h);
    const uint16_t* ob = seq_base<const uint16_t>(P.dout, p, x.b, x.e.q0, h);
    dmq.issue(make_rsrc(qb + (int64_t)qbase * P.q.ss, rows * qrb), st, wv);
    if constexpr (RPL > 0) {
      const bool graph = h < p.H_G;
      const uint16_t* sb = graph ? seq_base<const uint16_t>(P.rqs, p, x.b, x.e.q0, h) : qb;
      dmr.issue(make_rsrc(sb + (int64_t)qbase * P.rqs.ss, graph ? rows * srb : 0u), st + C::QB,
                wv);
    }
    dmo.issue(make_rsrc(ob + (int64_t)qbase * P.dout.ss, rows * orb), st + C::QB + C::RB, wv);
    const float* lb = is_delta ? seq_base<const float>(P.delta, p, x.b, x.e.q0, h)
                               : seq_base<const float>(P.nlse, p, x.b, x.e.q0, h);
    const int64_t lss = is_delta ? P.delta.ss : P.nlse.ss;
    const auto rl = make_rsrc(lb + (int64_t)qbase * lss, rows * (is_delta ? drb : lrb));
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        rl, (lds_void*)(st + C::QB + C::RB + C::OB + lslot), 4, loff, 0, 0, 0);
  };

  const TrLane tl(lane);
  const RowLane rdl(lane);

  auto compute = [&](const KvCursor& c, const uint8_t* cur) {
    const KvItem& x = c.it;
    const int h = x.kvh * p.group + c.hi;
    const bool graph = (RPL > 0) && (h < p.H_G);
    const int key = x.k0t + krow;
    const int wk0 = x.k0t + wv * 32;
    const int qbase = (x.qb_lo + c.qi) * C::BM;
    const bool active = wk0 < x.e.lk && (!p.causal || qbase + C::BM - 1 >= wk0);
    if (!active) return;
    const bool diag = p.causal && wk0 + 31 > qbase;
    const uint8_t* qt = cur;
    const uint8_t* rt = cur + C::QB;
    const uint8_t* ot = cur + C::QB + C::RB;
    const float* ls = (const float*)(cur + C::QB + C::RB + C::OB);
    const int nrs = graph ? cdiv(p.R, 16) : 0;
    bf16x8 pb[2][2], db[2][2];
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
      f32x16 sacc = f32x16{}, dpacc = f32x16{};
#pragma unroll
      for (int s = 0; s < C::KSD; ++s) sacc = mfma32(row_read<C::BM>(qt, rdl, rb * 32, s), kreg[s], sacc);
      if constexpr (C::KSR > 0) {
#pragma unroll
        for (int s = 0; s < C::KSR; ++s)
          if (s < nrs)
            sacc = mfma32(row_read<C::BM>(rt, rdl, rb * 32, s),
                          kreg[C::KSD + s], sacc);
      }
#pragma unroll
      for (int s = 0; s < C::KSD; ++s) dpacc = mfma32(row_read<C::BM>(ot, rdl, rb * 32, s), vreg[s], dpacc);
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
          const f32x4_t lse4 = *(const f32x4_t*)(ls + r0);  // -LSE log2(e)
          const f32x4_t dl4 = *(const f32x4_t*)(ls + C::BM + r0);
          float pv[4], dv[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int v = 4 * g + j;
            pv[j] = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[v], p.c2, lse4[j]));
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
          dvacc[d] = mfma32(tr_operand<C::BM>(ot, tl, k0, 32 * d), pb[rb][half], dvacc[d]);
#pragma unroll
        for (int f = 0; f < C::NDB; ++f)
          dkacc[f] = mfma32(tr_operand<C::BM>(qt, tl, k0, 32 * f), db[rb][half], dkacc[f]);
        if constexpr (C::NRB > 0) {
          if (graph) {
#pragma unroll
            for (int f = 0; f < C::NRB; ++f)
              dkacc[C::NDB + f] =
                  mfma32(tr_operand<C::BM>(rt, tl, k0, 32 * f), db[rb][half], dkacc[C::NDB + f]);
          }
        }
      }
  };

  KvCursor cc;  // compute cursor
  cc.r = -1;
  cc.done = false;
  next_item(cc, true);
  if (cc.done) return;
  load_kv(cc.it);
  load_rk(cc.it, cc.it.kvh * p.group);
#pragma unroll
  for (int i = 0; i < C::NDB; ++i) dvacc[i] = f32x16{};
#pragma unroll
  for (int i = 0; i < C::NDB + C::NRB; ++i) dkacc[i] = f32x16{};

  KvCursor ic = cc;  // issue cursor, two blocks ahead
  int pending = 1;
  issue(ic, st0);
  advance(ic, false);
  if (!ic.done) {
    issue(ic, st1);
    advance(ic, false);
    ++pending;
  }

  // One block: wait for its tiles, start the DMA two blocks ahead into
  // `nxt`, compute on `cur`; after an item's (head's) last block, write its
  // results and load the next item's (head's) stationary rows.
  auto step = [&](const uint8_t* cur, uint8_t* nxt) {
    if (pending == 2) ring_barrier<C::PER_STEP>(); else ring_barrier<0>();
    --pending;
    if (!ic.done) {
      issue(ic, nxt);
      advance(ic, false);
      ++pending;
    }
    __builtin_amdgcn_sched_barrier(0);
    compute(cc, cur);
    if (cc.qi + 1 < cc.it.nqb) {
      ++cc.qi;
      return;
    }
    // Keep the stores and the next item's loads after this block's MFMAs (the
    // old and new stationary rows must not be live at once).
    __builtin_amdgcn_sched_barrier(0);
    const KvItem x = cc.it;
    const bool last_head = cc.hi + 1 == p.group;
    write_drk(x, x.kvh * p.group + cc.hi, false);
    if (last_head) write_dkdv(x, false);
    advance(cc, true);
    if (cc.done) return;
    if (last_head) {
      load_kv(cc.it);
#pragma unroll
      for (int i = 0; i < C::NDB; ++i) dvacc[i] = f32x16{};
#pragma unroll
      for (int i = 0; i < C::NDB; ++i) dkacc[i] = f32x16{};
    }
    load_rk(cc.it, cc.it.kvh * p.group + cc.hi);
#pragma unroll
    for (int i = C::NDB; i < C::NDB + C::NRB; ++i) dkacc[i] = f32x16{};
  };

  for (;;) {
    step(st0, st2);
    if (cc.done) break;
    step(st1, st0);
    if (cc.done) break;
    step(st2, st1);
    if (cc.done) break;
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
