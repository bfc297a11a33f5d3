// fna2_bwd_dkdv.hip — dK, dV, dRk for gfx950.
//
// Replaces _fna2_bwd_dkdv_kernel / _fna2_bwd_dkdv_varlen_kernel
// (FNA2/flash_naylis_attn.py:390-553, :929-1076).
//
// Persistent: one workgroup per CU walks a list of work items, an item being
// the keys of one key tile (4 waves x KPW slices of 32) of one KV head;
// workgroup g takes items
// g, 2G-1-g, 2G+g, ... (snake order over a longest-first list).  For each
// query head of the GQA group an item walks the 32-query blocks that can see
// its keys (causal: from the key tile's diagonal on).
//
// The workgroup's 8 waves split the work by role, two waves per SIMD:
//   * producer wave w (0-3) keeps the K | Rk and V rows of its KPW slices of
//     32 keys in registers (B operands, one key per lane) and per block forms
//       S, dP  (32 x 32)               A operands: Q | Rq and dO rows
//       P = exp(S - LSE),  dS = P (dP - delta)
//     and stores P and dS, already in MFMA operand layout, to LDS;
//   * consumer wave 4 + w holds the fp32 accumulators of the same keys and,
//     one block behind, forms
//       dV^T  += dO^T P                A operand: dO^T by transpose reads
//       acc^T += [Q | Rq]^T dS         A operand: the same tiles transposed
//     and at the end of an item writes dK = a c acc_D, dRk = graph_scale[h]
//     acc_R (= graph_scale dS^T Rq) and dV straight from the accumulators
//     (one lane exchange per register pair makes 16-byte row pieces).
// A producer's softmax arithmetic thus overlaps its SIMD partner's MFMAs,
// and neither role needs more than half of the SIMD's registers.  dK and dV
// accumulate over the whole GQA group in fp32: no atomics.
//
// The dQ kernel stores delta and -LSE log2(e) (Rq is read where the caller
// holds it); the sign/zero factor a of the augmented query rides on the
// stationary K (exact), and S is formed as the forward forms it (the rank
// chain scaled by b = graph_scale[h] / c in fp32, then the head-dim chain),
// so the recomputed S equals the forward's bit for bit.
//
// Q, Rq, dO, -LSE log2(e) and delta tiles stream in by DMA through a
// four-stage ring that runs two blocks ahead of the producers, across item
// boundaries; the consumers read a stage one block later.  With two key
// slices per wave the consumers issue that DMA (right after their barrier:
// they idle while the producers compute), otherwise the producers do (the
// consumers' own step would then be the longer).  The last block of an
// (item, head) loads the rows of the next one into the registers its MFMAs
// have just read: V from memory, K | Rk from LDS tiles that the consumers
// DMA'd during the current one (where the LDS has room for them).  Both
// roles meet at one barrier per block.  The stages are separate LDS objects
// and the loops are unrolled by four so that the compiler can prove that
// reads and in-flight DMA never alias.
#include "fna2_kernels.h"
#include "fna2_tile.h"

namespace fna2 {

namespace {

enum : unsigned { kTileQ = 1, kTileR = 2, kTileO = 4, kTileL = 8, kTileAll = 15 };

// RS: 16-deep rank steps of the score chain (RPL / 16, or 1 where R <= 16:
// the second step of a 32-wide rank tile would multiply zeros).
template <int D, int RPL, bool F16, int RS>
struct KvCfg {
  static constexpr int NP = 4;       // producer waves (as many consumers)
  static constexpr int NW = 2 * NP;  // waves per workgroup
  static constexpr int KPW = kv_kpw(D, RPL);  // 32-key slices per wave
  static constexpr int BN = kv_bn(D, RPL);    // keys per item
  static constexpr int BM = kKvBM;            // queries per block
  static_assert(BM == 32 && BN == 32 * NP * KPW, "32 x 32 MFMA blocks");
  static constexpr int CD = D / 8;
  static constexpr int CR = RPL > 0 ? RPL / 8 : 4;
  static constexpr int KSD = D / 16;
  static constexpr int KSR = RS;
  static_assert(RS * 16 <= RPL && (RPL == 0) == (RS == 0), "rank steps within the rank tile");
  static constexpr int NDB = D / 32;
  static constexpr int NRB = RPL / 32;
  static constexpr int QB = BM * D * 2;
  static constexpr int RB = BM * RPL * 2;
  static constexpr int OB = BM * D * 2;
  static constexpr int LB = 2 * 256;  // -LSE log2(e), delta: one 64-lane dword DMA each
  static constexpr int STAGE = QB + RB + OB + LB;
  // A producer's P and dS operands of one block: per key slice, P and dS in
  // the element type (two 16-query k-halves each), and with fp16 elements
  // and a rank tile also dS in bf16 for the dRk chain (Rq is bf16).
  static constexpr bool DBR = F16 && RPL > 0;
  static constexpr int SL = (DBR ? 6 : 4) * 1024;  // bytes per key slice
  static constexpr int PW = KPW * SL;
  static constexpr int PDS = NP * PW;
  using DmaD = Dma<BM, CD, NP>;
  using DmaR = Dma<BM, CR, NP>;
  // K and Rk tiles of the next (item, head) in LDS, DMA'd by the consumer
  // waves, where the LDS holds them next to the ring (not at d = 128 with
  // rank 64).
  static constexpr int KRK = BN * CD * 16;
  static constexpr int KRR = RPL > 0 ? BN * CR * 16 : 0;
  static constexpr bool KR = 4 * STAGE + 2 * PDS + KRK + KRR <= 160 * 1024;
  using DmaKK = Dma<BN, CD, NP>;
  using DmaKR = Dma<BN, CR, NP>;
  // The ring tiles of a block: Q, the rank operand, dO and the -LSE log2(e)
  // / delta rows.  CDMA: those the consumer waves DMA (at the start of their
  // step); the producers DMA the rest (at the end of theirs).  With two key
  // slices per wave the consumers have the time for all of them.  With one,
  // at d = 128 and rank 64 (no K | Rk tiles for them to DMA) they take the
  // dO tile (c4 dK/dV -3%; the -LSE / delta rows as well: +4.5%); at rank
  // 32 their own step is the longer with any (c3 +2 to +4 us), and the
  // producers keep them.
  static constexpr unsigned CDMA = KPW == 2 ? kTileAll : (D == 128 && RPL == 64) ? kTileO : 0u;
  // VMEM instructions per wave and block for the tiles in mask m.
  static constexpr int nb_of(unsigned m) {
    return ((m & kTileQ) ? DmaD::PER_WAVE : 0) +
           ((m & kTileR) && RPL > 0 ? DmaR::PER_WAVE : 0) +
           ((m & kTileO) ? DmaD::PER_WAVE : 0) + ((m & kTileL) ? 1 : 0);
  }
  static constexpr int NBC = nb_of(CDMA);              // per consumer wave
  static constexpr int NBP = nb_of(kTileAll & ~CDMA);  // per producer wave
};

// Scheduling pattern for a region of n operands, each `per` LDS reads that
// feed `mper` MFMAs: `ahead` operands' reads are issued first, then the
// MFMAs of one operand and the reads of a later one alternate.  This bounds
// the registers held by operands in flight (the scheduler would otherwise
// hoist every read).
template <int N, int PER, int AHEAD, int MPER = 1>
__device__ __forceinline__ void pipe_lds_mfma() {
#pragma unroll
  for (int i = 0; i < AHEAD; ++i) __builtin_amdgcn_sched_group_barrier(0x100, PER, 0);
#pragma unroll
  for (int i = 0; i < N - AHEAD; ++i) {
    __builtin_amdgcn_sched_group_barrier(0x008, MPER, 0);
    __builtin_amdgcn_sched_group_barrier(0x100, PER, 0);
  }
#pragma unroll
  for (int i = 0; i < AHEAD; ++i) __builtin_amdgcn_sched_group_barrier(0x008, MPER, 0);
}

// The kernel's parameter block, re-read where it is used: the pointer is
// made opaque, so the loads are not hoisted out of the loops and the values
// are not held (or spilled) across them.  Used on the per-item paths only.
typedef const __attribute__((address_space(4))) BwdParams* ParamsPtr;
__device__ __forceinline__ ParamsPtr params_here() {
  ParamsPtr pp = (ParamsPtr)__builtin_amdgcn_kernarg_segment_ptr();
  asm volatile("" : "+s"(pp));
  return pp;
}
__device__ __forceinline__ TView view_of(const __attribute__((address_space(4))) TView* v) {
  TView t;
  t.ptr = v->ptr;
  t.sb = v->sb;
  t.ss = v->ss;
  t.sh = v->sh;
  return t;
}

struct KvItem {
  int b, kvh, k0t;  // sequence, KV head, first key of the tile
  SeqExt e;
  int qb_lo, nqb;   // first query block that sees the tile; blocks per head
};

// Position in a workgroup's program: item (round r), head hi, block qi.
struct KvCursor {
  int r, hi, qi;
  bool done;
  KvItem it;
};

// One role's share of the ring DMA: the tiles in MASK of a block, wave w of
// the role issuing exactly C::nb_of(MASK) VMEM instructions per block.
// Waves 0 and 2 of the role fetch the -LSE log2(e) row, 1 and 3 the delta
// row (the same bytes twice: every wave issues as many instructions).
template <class C, int RPL, unsigned MASK>
struct RingDma {
  typename C::DmaD dmq, dmo;
  typename C::DmaR dmr;
  uint32_t qrb, orb, srb, lrb, drb, loff;
  bool is_delta;
  // Buffer descriptors for the issue cursor's (item, head), set when it
  // enters one: they span the sequence's whole query range, so rows past it
  // read as zeros, and a block only adds its row offset to the lane
  // offsets.  (The host keeps a sequence's rows under 2 GB.)
  u32x4 sq, so, sr, sl;

  __device__ __forceinline__ void init(const BwdParams& P, int w, int lane) {
    qrb = (uint32_t)P.q.ss * 2u;
    orb = (uint32_t)P.dout.ss * 2u;
    srb = (uint32_t)P.rq.ss * 2u;
    if constexpr ((MASK & kTileQ) != 0) dmq.init_fixed(w, lane, qrb, C::CD);
    if constexpr ((MASK & kTileO) != 0) dmo.init_fixed(w, lane, orb, C::CD);
    // rank chunks past R read as zeros (past them lies the next head's rank)
    if constexpr ((MASK & kTileR) != 0 && RPL > 0) dmr.init_fixed(w, lane, srb, P.p.R / 8);
    is_delta = (w & 1) != 0;
    lrb = (uint32_t)P.nlse.ss * 4u;
    drb = (uint32_t)P.delta.ss * 4u;
    loff = (uint32_t)lane * (is_delta ? drb : lrb);
  }
  __device__ __forceinline__ void setup(const BwdParams& P, const KvCursor& c) {
    // Past the last block the ring's last DMAs read nothing (zero-size
    // descriptors); no branch, so that every descriptor stays in registers.
    const Problem& p = P.p;
    const bool done = uni((int)c.done) != 0;
    const int b = done ? 0 : c.it.b, q0 = done ? 0 : c.it.e.q0;
    const int h = done ? 0 : c.it.kvh * p.group + c.hi;
    const uint32_t lq = done ? 0u : (uint32_t)c.it.e.lq;
    const ParamsPtr pp = params_here();
    const uint16_t* qb = seq_base<const uint16_t>(view_of(&pp->q), p, b, q0, h);
    if constexpr ((MASK & kTileQ) != 0) sq = rsrc_words(qb, lq * qrb);
    if constexpr ((MASK & kTileO) != 0)
      so = rsrc_words(seq_base<const uint16_t>(view_of(&pp->dout), p, b, q0, h), lq * orb);
    if constexpr ((MASK & kTileR) != 0 && RPL > 0) {
      const bool graph = h < p.H_G;
      sr = rsrc_words(graph ? seq_base<const uint16_t>(view_of(&pp->rq), p, b, q0, h) : qb,
                      graph ? lq * srb : 0u);
    }
    if constexpr ((MASK & kTileL) != 0) {
      const float* lb = seq_base<const float>(is_delta ? view_of(&pp->delta) : view_of(&pp->nlse),
                                              p, b, q0, h);
      sl = rsrc_words(lb, lq * (is_delta ? drb : lrb));
    }
  }
  // Exactly C::nb_of(MASK) VMEM instructions, unconditionally.
  __device__ __forceinline__ void issue(const KvCursor& c, uint8_t* st, int w) const {
    const uint32_t q0 = c.done ? 0u : (uint32_t)((c.it.qb_lo + c.qi) * C::BM);
    if constexpr ((MASK & kTileQ) != 0) dmq.issue_fixed(sq, st, w, q0 * qrb);
    if constexpr ((MASK & kTileR) != 0 && RPL > 0) dmr.issue_fixed(sr, st + C::QB, w, q0 * srb);
    if constexpr ((MASK & kTileO) != 0) dmo.issue_fixed(so, st + C::QB + C::RB, w, q0 * orb);
    if constexpr ((MASK & kTileL) != 0)
      dma_lds<4>(sl, lds_addr(st + C::QB + C::RB + C::OB + (is_delta ? 256 : 0)),
                 loff + q0 * (is_delta ? drb : lrb));
  }
};

template <int D, int RPL, bool F16, int RS>
__device__ __forceinline__ void dkdv_body(const BwdParams& P) {
  using C = KvCfg<D, RPL, F16, RS>;
  __shared__ __attribute__((aligned(1024))) uint8_t st0[C::STAGE];
  __shared__ __attribute__((aligned(1024))) uint8_t st1[C::STAGE];
  __shared__ __attribute__((aligned(1024))) uint8_t st2[C::STAGE];
  __shared__ __attribute__((aligned(1024))) uint8_t st3[C::STAGE];
  __shared__ __attribute__((aligned(1024))) uint8_t pd0[C::PDS];
  __shared__ __attribute__((aligned(1024))) uint8_t pd1[C::PDS];
  __shared__ __attribute__((aligned(1024))) uint8_t krk[C::KR ? C::KRK : 16];
  __shared__ __attribute__((aligned(1024))) uint8_t krr[C::KR && RPL > 0 ? C::KRR : 16];
  const Problem& p = P.p;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = uni(tid >> 6);
  const int kw = wv & (C::NP - 1);  // keys of this wave: 32-key slices kw KPW ..
  const int l32 = lane & 31, hl = lane >> 5;
  // this lane's key within the item in the wave's slice j
  auto krow_of = [&](int j) { return (kw * C::KPW + j) * 32 + l32; };
  const int G = gridDim.x, g = blockIdx.x;
  const int n_items =
      (P.tiles_k ? min(uni(*const_space(P.n_tiles_k)), P.k_tiles) : p.nseq * cdiv(p.sk, C::BN)) *
      p.H_KV;

  auto decode = [&](int r) {
    KvItem x;
    const int w = r * G + ((r & 1) ? G - 1 - g : g);
    const int tix = w / p.H_KV;
    x.kvh = w - tix * p.H_KV;
    int kt;
    if (P.tiles_k) {
      tile_decode(P.tiles_k, tix, x.b, kt, x.e);
    } else {
      x.b = tix % p.nseq;
      kt = tix / p.nseq;
      x.e = seq_ext_uniform(p, x.b);
    }
    x.k0t = kt * C::BN;
    x.qb_lo = p.causal ? x.k0t / C::BM : 0;
    x.nqb = max(cdiv(x.e.lq, C::BM) - x.qb_lo, 0);
    return x;
  };
  auto round_valid = [&](int r) { return r * G + ((r & 1) ? G - 1 - g : g) < n_items; };

  // The program: items in snake order, then the heads of the GQA group, then
  // 32-query blocks.  An item no query block can see (keys past every query
  // under the causal mask, or an empty query range) has zero gradients;
  // on_zero is called as the cursor passes it.
  auto next_item = [&](KvCursor& c, auto&& on_zero) {
    for (;;) {
      ++c.r;
      if (!round_valid(c.r)) {
        c.done = true;
        return;
      }
      c.it = decode(c.r);
      c.hi = 0;
      c.qi = 0;
      if (c.it.nqb > 0) return;
      on_zero(c.it);
    }
  };
  auto advance = [&](KvCursor& c, auto&& on_zero) {
    if (++c.qi < c.it.nqb) return;
    c.qi = 0;
    if (++c.hi < p.group) return;
    next_item(c, on_zero);
  };
  auto start = [&](KvCursor& c, auto&& on_zero) {
    c.r = -1;
    c.done = false;
    next_item(c, on_zero);
  };
  auto no_zero = [](const KvItem&) {};
  // The first block of the (item, head) after the cursor's (lookahead only).
  auto next_seg = [&](KvCursor c) {
    c.qi = 0;
    if (++c.hi >= p.group) next_item(c, no_zero);
    return c;
  };
  // Whether this wave's keys meet block qi of the cursor's item.
  auto block_active = [&](const KvCursor& c) {
    const int wk0 = c.it.k0t + kw * 32 * C::KPW;
    const int qbase = (c.it.qb_lo + c.qi) * C::BM;
    return wk0 < c.it.e.lk && (!p.causal || qbase + C::BM - 1 >= wk0);
  };

  if (wv < C::NP) {
    // ============================ producers ============================
    const RowLane rdl(lane);
    // Stationary rows (B operands): lane holds key krow, features
    // 16s + 8hl .. +7 of k-step s: K | Rk and V of the producer's (item,
    // head), loaded in place (load16_inplace) and waited for by the ring
    // barrier.  Rank chunks past R (features R .. padded rank) are read at an
    // out-of-range offset, so the buffer unit returns zeros: they are never
    // read from memory (past R lie the next head's rank or, for the last row
    // of the last graph head, the end of R_k's allocation).
    u32x4 kreg[C::KPW][C::KSD + C::KSR], vreg[C::KPW][C::KSD];
#pragma unroll
    for (int j = 0; j < C::KPW; ++j) {
#pragma unroll
      for (int s = 0; s < C::KSD + C::KSR; ++s) kreg[j][s] = u32x4{0u, 0u, 0u, 0u};
#pragma unroll
      for (int s = 0; s < C::KSD; ++s) vreg[j][s] = u32x4{0u, 0u, 0u, 0u};
    }
    auto load_k = [&](const KvItem& x, int h, bool skip) {
      const ParamsPtr pp = params_here();
      const TView vk = view_of(&pp->k), vr = view_of(&pp->rk);
      const uint32_t krows = (uint32_t)max(min(C::BN, x.e.lk - x.k0t), 0);
      const uint32_t krb = (uint32_t)vk.ss * 2u;
      const uint32_t rrb = (uint32_t)vr.ss * 2u;
      const bool graph = h < p.H_G;
      const uint16_t* kb = seq_base<const uint16_t>(vk, p, x.b, x.e.k0, x.kvh);
      const uint16_t* rkb = graph ? seq_base<const uint16_t>(vr, p, x.b, x.e.k0, h) : kb;
      const u32x4 rk = rsrc_words(kb + (int64_t)x.k0t * vk.ss, krows * krb);
      const u32x4 rr = rsrc_words(rkb + (int64_t)x.k0t * vr.ss, graph ? krows * rrb : 0u);
      // skip: every offset out of range (the buffer unit returns zeros
      // without touching memory), so that this is one load site whichever
      // way the rows come
#pragma unroll
      for (int j = 0; j < C::KPW; ++j) {
        const uint32_t ko = skip ? kOOB : (uint32_t)krow_of(j) * krb + 16u * hl;
        const uint32_t ro = (uint32_t)krow_of(j) * rrb + 16u * hl;
        static_for<C::KSD>(
            [&](auto s) { load16_inplace<32 * decltype(s)::value>(kreg[j][s], rk, ko); });
        static_for<C::KSR>([&](auto s) {
          const bool in = !skip && (2 * decltype(s)::value + hl) * 8 < p.R;
          load16_inplace<32 * decltype(s)::value>(kreg[j][C::KSD + s], rr, in ? ro : kOOB);
        });
      }
    };
    auto load_v = [&](const KvItem& x) {
      const ParamsPtr pp = params_here();
      const TView vv = view_of(&pp->v);
      const uint32_t krows = (uint32_t)max(min(C::BN, x.e.lk - x.k0t), 0);
      const uint32_t vrb = (uint32_t)vv.ss * 2u;
      const uint16_t* vb = seq_base<const uint16_t>(vv, p, x.b, x.e.k0, x.kvh);
      const u32x4 rv = rsrc_words(vb + (int64_t)x.k0t * vv.ss, krows * vrb);
#pragma unroll
      for (int j = 0; j < C::KPW; ++j) {
        const uint32_t vo = (uint32_t)krow_of(j) * vrb + 16u * hl;
        static_for<C::KSD>(
            [&](auto s) { load16_inplace<32 * decltype(s)::value>(vreg[j][s], rv, vo); });
      }
    };
    // K | Rk rows of this wave's keys from the LDS tiles the consumers filled
    // (the row-read pattern of the tiles: chunk 2s + lane / 32 of row
    // kw * 32 + lane % 32).  In place, as every other write of these
    // registers, so that the compiler keeps them where the in-place global
    // loads put them; the explicit wait replaces the one it does not insert.
    auto read_kr = [&]() {
#pragma unroll
      for (int j = 0; j < C::KPW; ++j) {
        const uint32_t row = (uint32_t)((kw * C::KPW + j) * 32 * 64);
        const uint32_t kb0 = lds_addr(krk) + row + (uint32_t)rdl.off[0];
        const uint32_t kb1 = lds_addr(krk) + row + (uint32_t)rdl.off[1];
        static_for<C::KSD>([&](auto s) {
          constexpr int S = decltype(s)::value;
          ds_read16_inplace<(S >> 1) * C::BN * 64>(kreg[j][S], (S & 1) ? kb1 : kb0);
        });
        if constexpr (C::KSR > 0) {
          const uint32_t rb0 = lds_addr(krr) + row + (uint32_t)rdl.off[0];
          const uint32_t rb1 = lds_addr(krr) + row + (uint32_t)rdl.off[1];
          static_for<C::KSR>([&](auto s) {
            constexpr int S = decltype(s)::value;
            ds_read16_inplace<(S >> 1) * C::BN * 64>(kreg[j][C::KSD + S], (S & 1) ? rb1 : rb0);
          });
        }
      }
      __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
    };
    bool kr_in = false;  // the current (item, head)'s K | Rk wait in LDS
    // The streamed Q tile is raw, so the factor a in {1, -1, 0} of the
    // augmented operand goes on K (exact): Q (a K)^T = (a Q) K^T.
    const uint32_t kxor = p.qa < 0.f ? 0x80008000u : 0u;
    const uint32_t kand = p.qa == 0.f ? 0u : 0xffffffffu;
    auto sign_k = [&]() {
      if (p.qa != 1.f) {
#pragma unroll
        for (int j = 0; j < C::KPW; ++j)
#pragma unroll
          for (int s = 0; s < C::KSD; ++s)
#pragma unroll
            for (int i = 0; i < 4; ++i) kreg[j][s][i] = (kreg[j][s][i] & kand) ^ kxor;
      }
    };

    // b = graph_scale[h] / c of the producer's current head (0 for a vanilla
    // head), set when the cursor enters a head.
    float bhp = 0.f;
    auto head_scale = [&](const KvCursor& c) {
      const int h = c.it.kvh * p.group + c.hi;
      return uni_f(h < p.H_G ? *const_space(params_here()->gs + h) / p.c : 0.f);
    };

    // S (returned as the unmasked P = exp2(S c2 - LSE log2 e)) and dP of
    // this wave's key slices against block qi of the cursor.
    // The block's -LSE log2(e) and delta rows go to lsr (this lane's query
    // rows 8 gq + 4 hl .. +3, gq = 0..3: -LSE in lsr[gq], delta in
    // lsr[4 + gq]), read after the rank MFMAs so that their latency hides
    // under the S chain.
    auto scores = [&](const KvCursor& c, const uint8_t* cur, f32x16 (&sacc)[C::KPW],
                      f32x16 (&dpacc)[C::KPW], f32x4_t (&lsr)[8]) {
      // (A vanilla head, or rank padding, has zero rank operands: its rank
      // MFMAs add exact zeros and keep the block one basic block.)
      const uint8_t* qt = cur;
      const uint8_t* rt = cur + C::QB;
      const uint8_t* ot = cur + C::QB + C::RB;
      // All A operands are read first (the LDS latency is paid once per
      // block, not once per MFMA); S and dP chains interleave.
      bf16x8 qa[C::KSD + C::KSR], oa[C::KSD];
#pragma unroll
      for (int s = 0; s < C::KSD; ++s) qa[s] = row_read<C::BM>(qt, rdl, 0, s);
#pragma unroll
      for (int s = 0; s < C::KSR; ++s) qa[C::KSD + s] = row_read<C::BM>(rt, rdl, 0, s);
#pragma unroll
      for (int s = 0; s < C::KSD; ++s) oa[s] = row_read<C::BM>(ot, rdl, 0, s);
      const float* ls = (const float*)(cur + C::QB + C::RB + C::OB);
#pragma unroll
      for (int gq = 0; gq < 4; ++gq) {
        lsr[gq] = *(const f32x4_t*)(ls + 8 * gq + 4 * hl);
        lsr[4 + gq] = *(const f32x4_t*)(ls + 64 + 8 * gq + 4 * hl);
      }
      // S / c = b Rq Rk^T + Q (a K)^T: the rank chain, scaled by b in fp32,
      // then the head-dim chain on top; then the dP chain.
      // (Every operand read serves the wave's KPW key slices.)
#pragma unroll
      for (int j = 0; j < C::KPW; ++j) {
        sacc[j] = f32x16{};
        dpacc[j] = f32x16{};
      }
#pragma unroll
      for (int s = 0; s < C::KSR; ++s)
#pragma unroll
        for (int j = 0; j < C::KPW; ++j)
          sacc[j] = mfma32(qa[C::KSD + s], as_bf16x8(kreg[j][C::KSD + s]), sacc[j]);
      if constexpr (C::KSR > 0) {
#pragma unroll
        for (int j = 0; j < C::KPW; ++j) sacc[j] *= bhp;
      }
#pragma unroll
      for (int s = 0; s < C::KSD; ++s)
#pragma unroll
        for (int j = 0; j < C::KPW; ++j)
          sacc[j] = mfma_e<F16>(qa[s], as_bf16x8(kreg[j][s]), sacc[j]);
      // issue order: the operand reads, the rank MFMAs, the -LSE / delta
      // reads, then (after the scaling) the head-dim MFMAs of S.  (The -LSE
      // / delta reads with the operands instead: c2 / c5 dK/dV +2% with two
      // key slices, c3 +1.4 us and c4 +0.6% with one.)
      __builtin_amdgcn_sched_group_barrier(0x100, 2 * C::KSD + C::KSR, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, C::KSR * C::KPW, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, C::KSD * C::KPW, 0);
      __builtin_amdgcn_sched_barrier(0);
      // The dP chain, and between its MFMAs the exponentials of the finished
      // S chain, P = exp2(S c2 - LSE log2 e) in place (unmasked): they issue
      // while the dependent MFMAs run (against the two chains interleaved
      // and every exponential after both: c4 dK/dV -3%, c3 -1.5 us, c5 -1%).
      constexpr int EPS = 16 / C::KSD;  // exponentials per slice and k-step
#pragma unroll
      for (int s = 0; s < C::KSD; ++s) {
#pragma unroll
        for (int j = 0; j < C::KPW; ++j)
          dpacc[j] = mfma_e<F16>(oa[s], as_bf16x8(vreg[j][s]), dpacc[j]);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int j = 0; j < C::KPW; ++j)
#pragma unroll
          for (int u = 0; u < EPS; ++u) {
            const int v = EPS * s + u;
            sacc[j][v] = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[j][v], p.c2, lsr[v >> 2][v & 3]));
          }
        __builtin_amdgcn_sched_barrier(0);
      }
    };
    // P (the exponentials of scores, masked here on the causal diagonal) and
    // dS = P (dP - delta) to LDS in the B-operand layout
    // of the consumer's MFMAs: for k-half j (query rows 16j..16j+15), lane
    // (key l32, half hl) holds rows 16j + 8i + 4hl + e, i = 0..1, e = 0..3,
    // i.e. accumulator registers 8j..8j+7.
    auto softmax = [&](const KvCursor& c, uint8_t* pd, const f32x16 (&sacc_)[C::KPW],
                       const f32x16 (&dpacc_)[C::KPW], const f32x4_t (&lsr)[8]) {
      const KvItem& x = c.it;
      const int qbase = (x.qb_lo + c.qi) * C::BM;
#pragma unroll
      for (int ks = 0; ks < C::KPW; ++ks) {
      const f32x16& sacc = sacc_[ks];
      const f32x16& dpacc = dpacc_[ks];
      // Zero-filled query rows (past the sequence) have Q = dO = LSE =
      // delta = 0, so P (dP - delta) = 0 there; columns of keys past the
      // sequence are never stored.  Only the causal diagonal needs a mask:
      // query row qbase + r sees key k0t + krow iff r >= thr.  Blocks off
      // the diagonal (every block of a non-causal problem) skip the compare
      // and select, a fifth of the arithmetic per score.
      const bool diag = p.causal && x.k0t + (kw * C::KPW + ks) * 32 + 31 > qbase;  // wave-uniform
      const int thr = x.k0t + krow_of(ks) - qbase;
      auto body = [&](auto masked) {
        u32x4 pk[2], dk[2], dr[2];
#pragma unroll
        for (int gq = 0; gq < 4; ++gq) {
          const int r0 = 8 * gq + 4 * hl;
          const f32x4_t dl4 = lsr[4 + gq];
          float pv[4], dv[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int v = 4 * gq + j;
            const float e = sacc[v];
            if constexpr (decltype(masked)::value)
              pv[j] = r0 + j >= thr ? e : 0.f;
            else
              pv[j] = e;
            dv[j] = pv[j] * (dpacc[v] - dl4[j]);
          }
          pk[gq >> 1][2 * (gq & 1)] = pack_e<F16>(pv[0], pv[1]);
          pk[gq >> 1][2 * (gq & 1) + 1] = pack_e<F16>(pv[2], pv[3]);
          dk[gq >> 1][2 * (gq & 1)] = pack_e<F16>(dv[0], dv[1]);
          dk[gq >> 1][2 * (gq & 1) + 1] = pack_e<F16>(dv[2], dv[3]);
          if constexpr (C::DBR) {
            dr[gq >> 1][2 * (gq & 1)] = pack_bf16(dv[0], dv[1]);
            dr[gq >> 1][2 * (gq & 1) + 1] = pack_bf16(dv[2], dv[3]);
          }
        }
        uint8_t* o = pd + kw * C::PW + ks * C::SL + lane * 16;
        st16(o, pk[0]);
        st16(o + 1024, pk[1]);
        st16(o + 2048, dk[0]);
        st16(o + 3072, dk[1]);
        if constexpr (C::DBR) {
          st16(o + 4096, dr[0]);
          st16(o + 5120, dr[1]);
        }
      };
      if (diag)
        body(std::true_type{});
      else
        body(std::false_type{});
      }
    };

    // The producers' share of the ring: every step issues exactly C::NBP
    // VMEM instructions (their tiles of block T + 2), so "wait until C::NBP
    // are in flight" at step T's barrier waits for their tiles of block T
    // and everything issued before them, and nothing newer.  The rows of the
    // next (item, head) are loaded by the last block of the current one,
    // after its MFMAs and before its DMA, so the next step's barrier also
    // waits for them.  The DMA and the row loads are inline assembly, so the
    // compiler adds no wait of its own.
    RingDma<C, RPL, kTileAll & ~C::CDMA> ring;
    ring.init(P, wv, lane);
    KvCursor pc;  // the block being produced
    start(pc, no_zero);
    KvCursor ic = pc;  // the block whose tiles are issued next (two ahead)
    auto issue = [&](uint8_t* st) {
      if constexpr (C::NBP > 0) {
        ring.issue(ic, st, wv);
        if (!ic.done) {
          advance(ic, no_zero);
          if (ic.done || ic.qi == 0) ring.setup(P, ic);
        }
      }
    };
    if constexpr (C::NBP > 0) ring.setup(P, ic);
    if (!uni((int)pc.done)) {  // (uniform: no masked path around the loads)
      load_k(pc.it, pc.it.kvh * p.group + pc.hi, false);
      load_v(pc.it);
    }
    issue(st0);
    issue(st1);

    // Block T (stage `cur`): wait for its tiles; S, dP; at the last block of
    // an (item, head), load the next one's rows into the registers just
    // read; P, dS; start the producers' DMA of block T + 2.  (P and dS go
    // before the DMA: the DMA's issue can stall on the memory pipeline, and
    // the consumers wait for P and dS.)
    auto step = [&](const uint8_t* cur, uint8_t* nxt, uint8_t* pd) {
      ring_barrier<C::NBP>();
      if (pc.done) return;
      if (pc.qi == 0) {  // rows loaded by the previous block (or above)
        if constexpr (C::KR) {
          if (kr_in) read_kr();
          kr_in = false;
        }
        sign_k();
        bhp = head_scale(pc);
      }
      KvCursor nx = pc;
      advance(nx, no_zero);
      const bool act = block_active(pc);
      f32x16 sacc[C::KPW], dpacc[C::KPW];
      f32x4_t lsr[8];
      __builtin_amdgcn_sched_barrier(0);
      if (act) scores(pc, cur, sacc, dpacc, lsr);
      __builtin_amdgcn_sched_barrier(0);
      if (!nx.done && nx.qi == 0) {
        // The next (item, head)'s rows: after an (item, head) of two or more
        // blocks the consumers have DMA'd its K | Rk into LDS, and only V is
        // loaded here.
        // (One load site for each: branches around in-place loads of the
        // same registers made the compiler move them while in flight.)
        const bool from_lds = C::KR && pc.it.nqb >= 2;
        load_k(nx.it, nx.it.kvh * p.group + nx.hi, from_lds);
        load_v(nx.it);
        kr_in = from_lds;
      }
      __builtin_amdgcn_sched_barrier(0);
      if (act) softmax(pc, pd, sacc, dpacc, lsr);
      __builtin_amdgcn_sched_barrier(0);
      issue(nxt);
      __builtin_amdgcn_sched_barrier(0);
      pc = nx;
    };
    // Block T uses stage T % 4 and P/dS buffer T % 2.  Steps 0 .. nblocks-1
    // produce; one more meets the consumers' last barrier.
    for (;;) {
      bool last = pc.done;
      step(st0, st2, pd0);
      if (last) break;
      last = pc.done;
      step(st1, st3, pd1);
      if (last) break;
      last = pc.done;
      step(st2, st0, pd0);
      if (last) break;
      last = pc.done;
      step(st3, st1, pd1);
      if (last) break;
    }
  } else {
    // ============================ consumers ============================
    const TrLane tl(lane);
    f32x16 dvacc[C::KPW][C::NDB];
    f32x16 dkacc[C::KPW][C::NDB + C::NRB];
    static_for<C::KPW>([&](auto jj) {
      constexpr int j = decltype(jj)::value;
#pragma unroll
      for (int i = 0; i < C::NDB; ++i) dvacc[j][i] = f32x16{};
#pragma unroll
      for (int i = 0; i < C::NDB + C::NRB; ++i) dkacc[j][i] = f32x16{};
    });

    // dRk of head h = graph_scale[h] acc_R (zero: an item no query block sees).
    // Lane (key l32, half hl) holds features 32 t + 8 i + 4 hl + e of its key
    // in accumulator tile t; one exchange between the lane halves per
    // register pair (i = 2 u, 2 u + 1) gives each lane 8 consecutive
    // features: 32 t + 16 u + 8 hl .. +7, in the returned order.
    // (f16: std::bool_constant, rounding to fp16 rather than bf16)
    auto swap8 = [&](const f32x16& a, float sc, bool zero, int u, auto f16) {
      auto pk = [&](int v) {
        return zero ? 0u : pack_e<decltype(f16)::value>(sc * a[v], sc * a[v + 1]);
      };
      const auto lo = __builtin_amdgcn_permlane32_swap(pk(8 * u), pk(8 * u + 4), false, false);
      const auto hi = __builtin_amdgcn_permlane32_swap(pk(8 * u + 2), pk(8 * u + 6), false, false);
      return u32x4{lo[0], hi[0], lo[1], hi[1]};
    };
    auto write_drk = [&](const KvItem& x, int h, bool zero) {
      if constexpr (C::NRB > 0) {
        if (h < p.H_G) {
          const float sr = zero ? 0.f : *const_space(params_here()->gs + h);
          static_for<C::KPW>([&](auto jj) {
            constexpr int j = decltype(jj)::value;
            u32x4 w[C::NRB][2];
#pragma unroll
            for (int f = 0; f < C::NRB; ++f)
#pragma unroll
              for (int u = 0; u < 2; ++u)
                w[f][u] = swap8(dkacc[j][C::NDB + f], sr, zero, u, std::false_type{});
            const int key = x.k0t + krow_of(j);
            if (key < x.e.lk) {
              const TView vd = view_of(&params_here()->drk);
              uint16_t* rp =
                  seq_base<uint16_t>(vd, p, x.b, x.e.k0, h) + (int64_t)key * vd.ss + 8 * hl;
#pragma unroll
              for (int f = 0; f < C::NRB; ++f)
#pragma unroll
                for (int u = 0; u < 2; ++u)
                  if (32 * f + 16 * u + 8 * hl < p.R) *(u32x4*)(rp + 32 * f + 16 * u) = w[f][u];
            }
          });
        }
      }
    };
    // dK = a c acc_D and dV, 16 bytes per lane straight from the
    // accumulators: a store writes 32 contiguous bytes of each of the wave's
    // 32 rows.
    auto write_rows = [&](const KvItem& x, int j, const f32x16* acc, float sc, bool zero,
                          const TView& out) {
      u32x4 w[C::NDB][2];
#pragma unroll
      for (int t = 0; t < C::NDB; ++t)
#pragma unroll
        for (int u = 0; u < 2; ++u) w[t][u] = swap8(acc[t], sc, zero, u, std::bool_constant<F16>{});
      const int key = x.k0t + krow_of(j);
      if (key < x.e.lk) {
        uint16_t* rp = seq_base<uint16_t>(out, p, x.b, x.e.k0, x.kvh) + (int64_t)key * out.ss + 8 * hl;
#pragma unroll
        for (int t = 0; t < C::NDB; ++t)
#pragma unroll
          for (int u = 0; u < 2; ++u) *(u32x4*)(rp + 32 * t + 16 * u) = w[t][u];
      }
    };
    auto write_dk = [&](const KvItem& x, bool zero) {
      const ParamsPtr pp = params_here();
      static_for<C::KPW>([&](auto jj) {
        constexpr int j = decltype(jj)::value;
        write_rows(x, j, dkacc[j], p.qa * p.c, zero, view_of(&pp->dk));
      });
    };
    auto write_dv = [&](const KvItem& x, bool zero) {
      const ParamsPtr pp = params_here();
      static_for<C::KPW>([&](auto jj) {
        constexpr int j = decltype(jj)::value;
        write_rows(x, j, dvacc[j], 1.f, zero, view_of(&pp->dv));
      });
    };
    auto write_dkdv = [&](const KvItem& x, bool zero) {
      write_dk(x, zero);
      write_dv(x, zero);
    };
    auto on_zero = [&](const KvItem& x) {
      write_dkdv(x, true);
      for (int hi = 0; hi < p.group; ++hi) write_drk(x, x.kvh * p.group + hi, true);
    };

    // K | Rk of the (item, head) after the one whose first block is being
    // consumed, DMA'd into LDS for the producers' next switch.  This wave's
    // share of the two tiles; rows past the sequence and rank chunks past R
    // read as zeros.
    typename C::DmaKK dkk;
    typename C::DmaKR dkr;
    const uint32_t kkb = (uint32_t)P.k.ss * 2u, krb2 = (uint32_t)P.rk.ss * 2u;
    if constexpr (C::KR) {
      dkk.init_fixed(kw, lane, kkb, C::CD);
      if constexpr (RPL > 0) dkr.init_fixed(kw, lane, krb2, p.R / 8);
    }
    auto issue_kr = [&](const KvItem& x, int h) {
      const ParamsPtr pp = params_here();
      const TView vk = view_of(&pp->k), vr = view_of(&pp->rk);
      const uint32_t krows = (uint32_t)max(min(C::BN, x.e.lk - x.k0t), 0);
      const uint16_t* kb =
          seq_base<const uint16_t>(vk, p, x.b, x.e.k0, x.kvh) + (int64_t)x.k0t * vk.ss;
      dkk.issue_fixed(rsrc_words(kb, krows * kkb), krk, kw, 0u);
      if constexpr (RPL > 0) {
        const bool graph = h < p.H_G;
        const uint16_t* rb =
            graph ? seq_base<const uint16_t>(vr, p, x.b, x.e.k0, h) + (int64_t)x.k0t * vr.ss : kb;
        dkr.issue_fixed(rsrc_words(rb, graph ? krows * krb2 : 0u), krr, kw, 0u);
      }
    };

    // The consumers' share of the ring (C::NBC VMEM instructions per wave
    // and step): their tiles of block T + 2, DMA'd right after step T's
    // barrier, after the step's K | Rk DMA and before its stores.  Loads
    // complete in issue order, so "wait until C::NBC are in flight" before
    // the next barrier waits for their tiles of block T + 1 and every older
    // load (the K | Rk tiles included), whatever the stores.  Without a
    // share, the wave waits for its K | Rk DMA before the barrier at which
    // the producers switch to it.
    RingDma<C, RPL, C::CDMA> ring;
    ring.init(P, kw, lane);
    KvCursor ic;  // the block whose tiles are issued next
    auto issue = [&](uint8_t* st) {
      if constexpr (C::NBC > 0) {
        ring.issue(ic, st, kw);
        if (!ic.done) {
          advance(ic, no_zero);
          if (ic.done || ic.qi == 0) ring.setup(P, ic);
        }
      }
    };
    bool kr_issued = false;

    // (acc_R of a vanilla head is built from zero tiles and never stored.)
    auto consume = [&](const uint8_t* cur, const uint8_t* pd) {
      const uint8_t* qt = cur;
      const uint8_t* rt = cur + C::QB;
      const uint8_t* ot = cur + C::QB + C::RB;
      // Every transposed operand read serves the wave's KPW key slices.  One
      // slice reads its P and dS operands first; two read them one k-half
      // at a time (registers).
      // (dbrj: dS in bf16 for the dRk chain, where it differs from dbj)
      auto mfmas = [&](int j, const bf16x8* pbj, const bf16x8* dbj, const bf16x8* dbrj) {
#pragma unroll
        for (int d = 0; d < C::NDB; ++d) {
          const bf16x8 a = tr_operand<C::BM>(ot, tl, 16 * j, 32 * d);
#pragma unroll
          for (int ks = 0; ks < C::KPW; ++ks)
            dvacc[ks][d] = mfma_e<F16>(a, pbj[ks], dvacc[ks][d]);
        }
#pragma unroll
        for (int d = 0; d < C::NDB; ++d) {
          const bf16x8 a = tr_operand<C::BM>(qt, tl, 16 * j, 32 * d);
#pragma unroll
          for (int ks = 0; ks < C::KPW; ++ks)
            dkacc[ks][d] = mfma_e<F16>(a, dbj[ks], dkacc[ks][d]);
        }
#pragma unroll
        for (int f = 0; f < C::NRB; ++f) {
          const bf16x8 a = tr_operand<C::BM>(rt, tl, 16 * j, 32 * f);
#pragma unroll
          for (int ks = 0; ks < C::KPW; ++ks)
            dkacc[ks][C::NDB + f] = mfma32(a, dbrj[ks], dkacc[ks][C::NDB + f]);
        }
      };
      const uint8_t* o = pd + kw * C::PW + lane * 16;
      constexpr int NPD = C::DBR ? 3 : 2;  // operand reads per k-half and slice
      if constexpr (C::KPW == 1) {
        bf16x8 pb[2][1], db[2][1], dbr[2][1];
        pb[0][0] = as_bf16x8(ld16(o));
        pb[1][0] = as_bf16x8(ld16(o + 1024));
        db[0][0] = as_bf16x8(ld16(o + 2048));
        db[1][0] = as_bf16x8(ld16(o + 3072));
        if constexpr (C::DBR) {
          dbr[0][0] = as_bf16x8(ld16(o + 4096));
          dbr[1][0] = as_bf16x8(ld16(o + 5120));
        }
        mfmas(0, pb[0], db[0], C::DBR ? dbr[0] : db[0]);
        mfmas(1, pb[1], db[1], C::DBR ? dbr[1] : db[1]);
        __builtin_amdgcn_sched_group_barrier(0x100, 2 * NPD, 0);
        pipe_lds_mfma<2 * (2 * C::NDB + C::NRB), 2, 3>();
      } else {
        // Two key slices: per k-half j, the P / dS operands and the first
        // A transposed operands are read, then each MFMA pair's operand is
        // read A operands ahead, behind scheduling fences (the compiler's
        // own order, group barriers notwithstanding, waited for 9 of the 20
        // reads just issued: c2 dK/dV 115.6 -> 112.6 us, c5 421 -> 413;
        // three ahead instead of two: c2 -1.9%, c5 -0.5%; four: no better).
        constexpr int NO = 2 * C::NDB + C::NRB, A = 3;
        auto opnd = [&](int j, int r) {
          return r < C::NDB ? tr_operand<C::BM>(ot, tl, 16 * j, 32 * r)
                 : r < 2 * C::NDB ? tr_operand<C::BM>(qt, tl, 16 * j, 32 * (r - C::NDB))
                                  : tr_operand<C::BM>(rt, tl, 16 * j, 32 * (r - 2 * C::NDB));
        };
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          bf16x8 pbj[C::KPW], dbj[C::KPW], dbrj[C::KPW];
#pragma unroll
          for (int ks = 0; ks < C::KPW; ++ks) {
            pbj[ks] = as_bf16x8(ld16(o + ks * C::SL + j * 1024));
            dbj[ks] = as_bf16x8(ld16(o + ks * C::SL + 2048 + j * 1024));
            if constexpr (C::DBR) dbrj[ks] = as_bf16x8(ld16(o + ks * C::SL + 4096 + j * 1024));
          }
          bf16x8 ar[A];
#pragma unroll
          for (int r = 0; r < A; ++r) ar[r] = opnd(j, r);
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int r = 0; r < NO; ++r) {
            const bf16x8 a = ar[r % A];
            if (r + A < NO) ar[r % A] = opnd(j, r + A);
#pragma unroll
            for (int ks = 0; ks < C::KPW; ++ks) {
              if (r < C::NDB)
                dvacc[ks][r] = mfma_e<F16>(a, pbj[ks], dvacc[ks][r]);
              else if (r < 2 * C::NDB)
                dkacc[ks][r - C::NDB] = mfma_e<F16>(a, dbj[ks], dkacc[ks][r - C::NDB]);
              else
                dkacc[ks][r - C::NDB] = mfma32(a, C::DBR ? dbrj[ks] : dbj[ks], dkacc[ks][r - C::NDB]);
            }
            __builtin_amdgcn_sched_barrier(0);
          }
        }
      }
    };

    // Tiles of blocks 0 and 1.
    start(ic, no_zero);
    if constexpr (C::NBC > 0) ring.setup(P, ic);
    issue(st0);
    issue(st1);

    // The last workgroup's consumers also reduce the dQ kernel's d_gs
    // partials (complete: that kernel ran before this one), before their
    // first block.
    if (g == G - 1 && p.H_G > 0) reduce_dgs_waves(P, kw, C::NP, lane);

    KvCursor cc;  // the block being consumed
    start(cc, on_zero);
    // Step t consumes block t - 1 (nothing at t = 0).  The barrier does not
    // wait for the consumers' own stores.
    //
    // An item's dV is stored at the start of the next step, not with its
    // dK: the step that ends an item is the consumers' longest (its stores)
    // while the producers start the next item, and the one after it is the
    // producers' longest while the consumers have one block to consume.
    bool first = true;
    bool dv_pending = false;
    KvItem dv_item{};
    auto flush_dv = [&]() {
      if (dv_pending) {
        write_dv(dv_item, false);
        static_for<C::KPW>([&](auto jj) {
          constexpr int j = decltype(jj)::value;
#pragma unroll
          for (int i = 0; i < C::NDB; ++i) dvacc[j][i] = f32x16{};
        });
        dv_pending = false;
      }
    };
    auto step = [&](const uint8_t* cur, uint8_t* pd, uint8_t* nxt) {
      if constexpr (C::KR && C::NBC == 0) {
        // The producers switch to the next (item, head) at this step and
        // read its K | Rk from LDS after the barrier: this wave's DMA of it
        // must be complete.
        if (kr_issued && !first && !cc.done && cc.qi + 1 == cc.it.nqb) {
          __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0)
          kr_issued = false;
        }
      }
      ring_barrier<(C::NBC > 0 ? C::NBC : 63)>();
      if constexpr (C::KR) {
        // At the first block of an (item, head) of two or more blocks (the
        // producers read its K | Rk before this step's barrier); the
        // producers read the next one after the next barrier at the earliest.
        if (!first && !cc.done && cc.qi == 0 && cc.it.nqb >= 2) {
          const KvCursor ny = next_seg(cc);
          if (!ny.done) {
            issue_kr(ny.it, ny.it.kvh * p.group + ny.hi);
            kr_issued = true;
          }
        }
      }
      issue(nxt);
      if (first) {
        first = false;
        return;
      }
      flush_dv();
      if (cc.done) return;
      if (block_active(cc)) consume(cur, pd);
      if (cc.qi + 1 < cc.it.nqb) {
        ++cc.qi;
        return;
      }
      __builtin_amdgcn_sched_barrier(0);
      const KvItem x = cc.it;
      const bool last_head = cc.hi + 1 == p.group;
      write_drk(x, x.kvh * p.group + cc.hi, false);
      if (last_head) {
        write_dk(x, false);
        dv_pending = true;
        dv_item = x;
      }
      static_for<C::KPW>([&](auto jj) {
        constexpr int j = decltype(jj)::value;
#pragma unroll
        for (int i = C::NDB; i < C::NDB + C::NRB; ++i) dkacc[j][i] = f32x16{};
        if (last_head) {
#pragma unroll
          for (int i = 0; i < C::NDB; ++i) dkacc[j][i] = f32x16{};
        }
      });
      advance(cc, on_zero);
    };
    // Stage and P/dS buffer of block t - 1: st[(t + 3) % 4], pd[(t + 1) % 2];
    // the DMA of block t + 2 goes to st[(t + 2) % 4], which the consumers
    // read last at step t - 1 and the producers at step t - 2.
    for (;;) {
      step(st3, pd1, st2);
      if (cc.done) break;
      step(st0, pd0, st3);
      if (cc.done) break;
      step(st1, pd1, st0);
      if (cc.done) break;
      step(st2, pd0, st1);
      if (cc.done) break;
    }
    flush_dv();  // the last item's dV
    __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0): no DMA in flight at exit
  }
}

// One non-template kernel per (D, rank, element type) so that each has a
// host stub.  Rank names: 0, 32 and 64 are the padded rank tiles; 16 is the
// 32-wide tile with one rank step (R <= 16).
#define FNA2_DKDV_KERNEL(D, RNAME, RPL, RS)                                              \
  __global__ __launch_bounds__(512, 1) void dkdv_kernel_d##D##_r##RNAME(const BwdParams P) { \
    dkdv_body<D, RPL, false, RS>(P);                                                     \
  }                                                                                      \
  __global__ __launch_bounds__(512, 1) void dkdv_kernel_d##D##_r##RNAME##_f16(             \
      const BwdParams P) {                                                               \
    dkdv_body<D, RPL, true, RS>(P);                                                      \
  }
FNA2_DKDV_KERNEL(64, 0, 0, 0)
FNA2_DKDV_KERNEL(64, 16, 32, 1)
FNA2_DKDV_KERNEL(64, 32, 32, 2)
FNA2_DKDV_KERNEL(64, 64, 64, 4)
FNA2_DKDV_KERNEL(128, 0, 0, 0)
FNA2_DKDV_KERNEL(128, 16, 32, 1)
FNA2_DKDV_KERNEL(128, 32, 32, 2)
FNA2_DKDV_KERNEL(128, 64, 64, 4)
#undef FNA2_DKDV_KERNEL

}  // namespace

hipError_t launch_bwd_dkdv(const BwdParams& P, int rpl, int grid, hipStream_t s) {
  if (grid <= 0) return hipSuccess;
  void (*k)(const BwdParams) = nullptr;
  const bool r16 = rpl == 32 && P.p.R <= 16;  // one rank step
  if (P.p.f16) {
    if (P.p.D == 64)
      k = rpl == 0 ? dkdv_kernel_d64_r0_f16
          : rpl == 32 ? (r16 ? dkdv_kernel_d64_r16_f16 : dkdv_kernel_d64_r32_f16)
                      : dkdv_kernel_d64_r64_f16;
    if (P.p.D == 128)
      k = rpl == 0 ? dkdv_kernel_d128_r0_f16
          : rpl == 32 ? (r16 ? dkdv_kernel_d128_r16_f16 : dkdv_kernel_d128_r32_f16)
                      : dkdv_kernel_d128_r64_f16;
  } else {
    if (P.p.D == 64)
      k = rpl == 0 ? dkdv_kernel_d64_r0
          : rpl == 32 ? (r16 ? dkdv_kernel_d64_r16 : dkdv_kernel_d64_r32) : dkdv_kernel_d64_r64;
    if (P.p.D == 128)
      k = rpl == 0 ? dkdv_kernel_d128_r0
          : rpl == 32 ? (r16 ? dkdv_kernel_d128_r16 : dkdv_kernel_d128_r32) : dkdv_kernel_d128_r64;
  }
  if (!k || (rpl != 0 && rpl != 32 && rpl != 64)) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k, dim3(grid), dim3(512), 0, s, P);
  return hipGetLastError();
}

}  // namespace fna2
