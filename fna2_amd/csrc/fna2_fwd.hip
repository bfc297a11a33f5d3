// fna2_fwd.hip — FlashNaylisAttention-2 forward for gfx950.
//
// Replaces _fna2_fwd_kernel / _fna2_fwd_varlen_kernel
// (FNA2/flash_naylis_attn.py:58-201, :208-349).
//
// One workgroup = 4 waves = 128 queries of one (sequence, head); wave w owns
// queries 32w..32w+31 and keeps its augmented query operand [a Q | Rq]
// in registers.  Per key step (64 keys at d = 64, 32 at d = 128) the wave
// computes the transposed score tile S^T = Ka Qa^T (keys x 32 queries) with
// one MFMA chain over the augmented width D + R (the bias is fused into the
// same contraction), so
// each lane holds one query column and the row softmax needs one exchange
// (lane ^ 32).  The probabilities, rounded to the element type (bf16, or
// fp16 for fp16 q/k/v, as the reference's p.to(v.dtype), :187), are the B
// operand of O^T += V^T P^T straight from the accumulator registers; V^T comes from
// the row-major V tile through ds_read_b64_tr_b16.  K, Rk and V tiles are
// DMA'd global -> LDS (buffer_load ... lds, zero-filled past the sequence)
// into a two-stage ring: the next tile streams in while this one computes.
// At d = 128 the 32-key step keeps a wave within 168 registers and a
// workgroup within 40 KB of LDS, so three workgroups share a CU and cover
// each other's row-load and DMA latency (two at 64 keys); at d = 64 the
// 64-key step already leaves room for more.
#include "fna2_kernels.h"
#include "fna2_tile.h"

namespace fna2 {

namespace {

template <int D, int RPL>
struct FwdCfg {
  static constexpr int NW = 4;
  static constexpr int BM = kFwdBM;
  static constexpr int BN = D == 128 ? 32 : kFwdBN;  // keys per step
  static constexpr int CD = D / 8;      // chunks per K / V row
  static constexpr int CR = RPL / 8;    // chunks per Rk row (0 without graph heads)
  static constexpr int KSD = D / 16;    // 16-deep steps over the head dim
  static constexpr int KSR = RPL / 16;  // ... over the (padded) rank
  static constexpr int KBYTES = BN * D * 2;
  static constexpr int RBYTES = BN * RPL * 2;
  static constexpr int VBYTES = BN * D * 2;
  static constexpr int STAGE = KBYTES + RBYTES + VBYTES;
  // Rank tile <= 32: K operand reads in flight kAhead k-steps ahead of the
  // S MFMAs (the register budget of three waves per SIMD at d = 128, four
  // at d = 64, leaves room for two; none at rank 64).  V^T operands
  // kAhead2 MFMAs ahead of the O MFMAs: two, one at rank 64.
  static constexpr bool PIPE = RPL <= 32;
  static constexpr int kAhead = 2;
  static constexpr int kAhead2 = PIPE ? 2 : 1;
};

// S16 (R <= 16, rank tile 32): the rank chain accumulates b <Rq, Rk>
// directly.  The query's rank operand holds b Rq split in two bf16 parts,
// hi = bf16(b Rq) in features 0..15 and lo = bf16(b Rq - hi) in features
// 16..31 of the tile, and the key-side tile holds Rk in both halves (its DMA
// mirrors chunks 0..1 into 2..3): the two 16-deep rank steps then sum to
// <hi + lo, Rk>, b <Rq, Rk> to 2^-16 (the products exact in fp32), and the
// score tile needs no scaling by b -- 16 VALU multiplies fewer per 32 x 32
// tile for one more MFMA, and no register more (the halves are the padding
// of the rank tile).
template <int D, int RPL, bool F16, bool S16>
__device__ __forceinline__ void fwd_body(const FwdParams& P) {
  using C = FwdCfg<D, RPL>;
  static_assert(!S16 || RPL == 32, "the split uses the padding of a 32-wide rank tile");
  // Two stages as separate objects: the compiler can then tell that reads of
  // one stage never alias the DMA into the other and does not wait for it.
  __shared__ __attribute__((aligned(1024))) uint8_t stage0[C::STAGE];
  __shared__ __attribute__((aligned(1024))) uint8_t stage1[C::STAGE];
  const Problem& p = P.p;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (scalar)
  const int l32 = lane & 31, hl = lane >> 5;
  const int h = blockIdx.x % p.H;
  const int tix = blockIdx.x / p.H;
  int b, qt;
  SeqExt e;
  if (P.tiles) {
    if (tix >= uni(*const_space(P.n_tiles))) return;
    tile_decode(P.tiles, tix, b, qt, e);
  } else {
    const int nqt = cdiv(p.sq, C::BM);
    b = tix % p.nseq;
    qt = nqt - 1 - tix / p.nseq;  // longest causal tiles first
    e = seq_ext_uniform(p, b);
  }
  const int kvh = h / p.group;
  const bool graph = (RPL > 0) && (h < p.H_G);
  const float bh = uni_f(graph ? *const_space(P.gs + h) / p.c : 0.f);
  // The rank MFMAs run unconditionally: rank features past R and a vanilla
  // head's rank operands are zeros on both sides (its rank tiles are DMA'd
  // from a zero-size range).  A branch around them made the compiler zero
  // the accumulator registers before it (at d = 128 c4 forward -2%; at
  // d = 64, with the operand reads ahead, c5 forward -2%).

  const uint16_t* qb = seq_base<const uint16_t>(P.q, p, b, e.q0, h);
  const uint16_t* kb = seq_base<const uint16_t>(P.k, p, b, e.k0, kvh);
  const uint16_t* vb = seq_base<const uint16_t>(P.v, p, b, e.k0, kvh);

  const int q0 = qt * C::BM;                 // first query of the tile
  const int qrow = q0 + wv * 32 + l32;       // this lane's query
  const bool qvalid = qrow < e.lq;
  const int wq0 = q0 + wv * 32;
  const int wq_last = min(wq0 + 31, e.lq - 1);
  const int qrows = max(min(C::BM, e.lq - q0), 0);

  int kv_hi = e.lk;
  if (p.causal) kv_hi = min(kv_hi, min(e.lq, q0 + C::BM));
  const int nkv = cdiv(max(kv_hi, 0), C::BN);

  // DMA plans (lane offsets are tile-invariant; descriptors move per tile).
  const uint32_t krb = (uint32_t)P.k.ss * 2u, vrb = (uint32_t)P.v.ss * 2u;
  Dma<C::BN, C::CD, C::NW> dk, dv;
  dk.init(wv, lane, krb, C::CD);
  dv.init(wv, lane, vrb, C::CD);
  Dma<C::BN, (C::CR > 0 ? C::CR : 4), C::NW> dr;
  uint32_t rkrb = 0;
  const uint16_t* rkb = kb;
  if constexpr (C::CR > 0) {
    rkrb = (uint32_t)P.rk.ss * 2u;
    if (graph) rkb = seq_base<const uint16_t>(P.rk, p, b, e.k0, h);
    dr.init(wv, lane, rkrb, p.R / 8, S16);
  }
  auto issue = [&](int kt, uint8_t* base) {
    const int k0 = kt * C::BN;
    const uint32_t rows = (uint32_t)max(min(C::BN, e.lk - k0), 0);
    dk.issue(make_rsrc(kb + (int64_t)k0 * P.k.ss, rows * krb), base, wv);
    if constexpr (C::CR > 0) {
      // (a vanilla head's rank tile is a zero-size range: the DMA writes
      // zeros and its rank MFMAs add exact zeros)
      dr.issue(make_rsrc(rkb + (int64_t)k0 * P.rk.ss, graph ? rows * rkrb : 0u), base + C::KBYTES,
               wv);
    }
    dv.issue(make_rsrc(vb + (int64_t)k0 * P.v.ss, rows * vrb), base + C::KBYTES + C::RBYTES, wv);
  };

  // The first key tile's DMA goes out before the query loads below, so the
  // two latencies overlap instead of adding up.
  if (nkv > 0) issue(0, stage0);
  __builtin_amdgcn_sched_barrier(0);

  // Query operand (B of S^T): lane holds Qa[qrow][16s + 8hl .. +7].
  bf16x8 qreg[C::KSD + C::KSR];
  {
    const uint32_t rb = (uint32_t)P.q.ss * 2u;
    const auto rs = make_rsrc(qb + (int64_t)q0 * P.q.ss, (uint32_t)qrows * rb);
    const uint32_t vo = (uint32_t)(wv * 32 + l32) * rb + (uint32_t)(16 * hl);
    const uint32_t qxor = p.qa < 0.f ? 0x80008000u : 0u;
    const uint32_t qand = p.qa == 0.f ? 0u : 0xffffffffu;
#pragma unroll
    for (int s = 0; s < C::KSD; ++s)
      qreg[s] = as_bf16x8(__builtin_amdgcn_raw_buffer_load_b128(rs, vo + 32u * s, 0, 0));
    // a Q (sign, or zero for a zero scale).  At d = 128 only where a != 1:
    // the sign and mask need the loaded rows, and waiting for them holds
    // the rank rows' loads below back by a round trip to memory (c3 forward
    // -0.9 us, c4 -0.7%).  At d = 64 that wait measured faster (c2 +1.1 us
    // without it: its single round of workgroups issues every row at once),
    // and so it stays.
    if (D == 64 || p.qa != 1.f) {
#pragma unroll
      for (int s = 0; s < C::KSD; ++s) {
        u32x4 v = as_u32x4(qreg[s]);
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = (v[i] & qand) ^ qxor;
        qreg[s] = as_bf16x8(v);
      }
    }
    if constexpr (C::KSR > 0) {
      const uint32_t rrb = (uint32_t)P.rq.ss * 2u;
      const uint16_t* rqb = graph ? seq_base<const uint16_t>(P.rq, p, b, e.q0, h) : qb;
      const auto rr = make_rsrc(rqb + (int64_t)q0 * P.rq.ss, graph ? (uint32_t)qrows * rrb : 0u);
      const uint32_t ro = (uint32_t)(wv * 32 + l32) * rrb + (uint32_t)(16 * hl);
#pragma unroll
      for (int s = 0; s < C::KSR; ++s) {
        const bool in = (2 * s + hl) * 8 < p.R;
        qreg[C::KSD + s] =
            as_bf16x8(__builtin_amdgcn_raw_buffer_load_b128(rr, in ? ro + 32u * s : kOOB, 0, 0));
      }
      if constexpr (S16) {
        // this lane's features 8 hl .. +7 (step 0): hi there, lo in step 1
        const u32x4 r = as_u32x4(qreg[C::KSD]);
        u32x4 hi, lo;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float x0 = bf16_lo(r[i]) * bh, x1 = bf16_hi(r[i]) * bh;
          hi[i] = pack_bf16(x0, x1);
          lo[i] = pack_bf16(x0 - bf16_lo(hi[i]), x1 - bf16_hi(hi[i]));
        }
        qreg[C::KSD] = as_bf16x8(hi);
        qreg[C::KSD + 1] = as_bf16x8(lo);
      }
    }
  }

  f32x16 oacc[D / 32];
#pragma unroll
  for (int d = 0; d < D / 32; ++d) oacc[d] = f32x16{};
  float m_i = kNegInf, l_i = 0.f;
  const TrLane tl(lane);
  const RowLane rdl(lane);

  // One key tile: wait for its DMA, start the next one into the other stage,
  // then compute on this one.
  auto step = [&](int kt, const uint8_t* cur, uint8_t* nxt) {
    ring_barrier<0>();
    if (kt + 1 < nkv) issue(kt + 1, nxt);
    __builtin_amdgcn_sched_barrier(0);  // keep the whole prefetch ahead of the compute
    const int kbase = kt * C::BN;
    const bool active = (wq0 <= wq_last) && (!p.causal || kbase <= wq_last);
    if (!active) return;
    const uint8_t* kl = cur;
    const uint8_t* rl = kl + C::KBYTES;
    const uint8_t* vl = rl + C::RBYTES;
    // S^T / c = b Rk Rq^T + K (a Q)^T per 32-key block: the rank chain
    // first (exact bf16 products, fp32 sums), its accumulator scaled by b in
    // fp32, then the head-dim chain added on top.
    f32x16 sacc[C::BN / 32];
#pragma unroll
    for (int kb2 = 0; kb2 < C::BN / 32; ++kb2) {
      f32x16 acc = f32x16{};
      constexpr int A = C::PIPE ? C::kAhead : 1;
      bf16x8 kr[A];
      if constexpr (C::PIPE) {
#pragma unroll
        for (int s = 0; s < A; ++s) kr[s] = row_read<C::BN>(kl, rdl, kb2 * 32, s);
        __builtin_amdgcn_sched_barrier(0);
      }
      if constexpr (C::KSR > 0) {
#pragma unroll
        for (int s = 0; s < C::KSR; ++s)
          acc = mfma32(row_read<C::BN>(rl, rdl, kb2 * 32, s), qreg[C::KSD + s], acc);
        if constexpr (!S16) acc *= here_s(bh);
      }
      if constexpr (C::PIPE) {
        // the K operand reads A k-steps ahead of the MFMAs (issued before
        // the rank chain; the scheduling fences keep every read where it is
        // issued, else the compiler, short of registers, reads each operand
        // just before its MFMA and waits for it)
#pragma unroll
        for (int s = 0; s < C::KSD; ++s) {
          acc = mfma_e<F16>(kr[s % A], qreg[s], acc);
          if (s + A < C::KSD) kr[s % A] = row_read<C::BN>(kl, rdl, kb2 * 32, s + A);
          __builtin_amdgcn_sched_barrier(0);
        }
      } else {
#pragma unroll
        for (int s = 0; s < C::KSD; ++s)
          acc = mfma_e<F16>(row_read<C::BN>(kl, rdl, kb2 * 32, s), qreg[s], acc);
      }
      sacc[kb2] = acc;
    }
    if ((kbase + C::BN > e.lk) || (p.causal && kbase + C::BN - 1 > wq0)) {
#pragma unroll
      for (int kb2 = 0; kb2 < C::BN / 32; ++kb2)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int key = kbase + kb2 * 32 + 8 * (v >> 2) + 4 * hl + (v & 3);
          const bool dead = key >= e.lk || (p.causal && key > qrow);
          sacc[kb2][v] = dead ? kNegInf : sacc[kb2][v];
        }
    }
    float mx = kNegInf;
#pragma unroll
    for (int kb2 = 0; kb2 < C::BN / 32; ++kb2)
#pragma unroll
      for (int v = 0; v < 16; ++v) mx = fmaxf(mx, sacc[kb2][v]);
    mx = wave_pair_max(mx);
    // Lazy rescale: the running maximum m_i moves (and O, l are rescaled)
    // only when some query's maximum has grown by more than 8 in exp2 units.
    // Otherwise the stale m_i stays: P <= 2^8, which bf16 and fp32 hold with
    // the same relative precision, and O / l and the LSE come out the same
    // (up to the 1e-6 of the normaliser).  Past the first key tile the
    // rescale is then rare.
    if (__builtin_amdgcn_ballot_w64((mx - m_i) * p.c2 > 8.f) != 0) {
      const float m_new = fmaxf(m_i, mx);
      const float alpha = __builtin_amdgcn_exp2f((m_i - ((m_new == kNegInf) ? 0.f : m_new)) * p.c2);
      l_i *= alpha;
#pragma unroll
      for (int d = 0; d < D / 32; ++d) oacc[d] *= alpha;
      m_i = m_new;
    }
    const float nm = -((m_i == kNegInf) ? 0.f : m_i) * p.c2;
    float ls = 0.f;
    bf16x8 pb[C::BN / 16];
    u32x4 pk[C::BN / 16];
    // pairs i0 .. i1 - 1 of P operand q (16 keys: accumulator kb2 = q / 2,
    // registers 8 (q % 2) .. +7)
    auto exps = [&](int q, int i0, int i1) {
#pragma unroll
      for (int i = i0; i < i1; ++i) {
        const int v0 = 8 * (q & 1) + 2 * i;
        const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[q >> 1][v0], p.c2, nm));
        const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[q >> 1][v0 + 1], p.c2, nm));
        ls += p0 + p1;
        pk[q][i] = pack_e<F16>(p0, p1);
      }
      if (i1 == 4) pb[q] = as_bf16x8(pk[q]);
    };
    // O^T += V^T P^T, with the exponentials of P operand s + 1 between the
    // MFMAs of operand s, where they hide the MFMAs' operand reads (c5
    // forward -1.3%; at rank 64, where the compiler read each operand just
    // before its MFMA, c4 -1.1% with the reads one MFMA ahead)
    {
      constexpr int A = C::kAhead2, NS = C::BN / 16, N = NS * (D / 32), PPM = 4 / (D / 32);
      exps(0, 0, 4);
      bf16x8 vr[A];
#pragma unroll
      for (int i = 0; i < A; ++i) vr[i] = tr_operand<C::BN>(vl, tl, 16 * (i / (D / 32)), 32 * (i % (D / 32)));
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < N; ++i) {
        const int s = i / (D / 32), d = i % (D / 32);
        oacc[d] = mfma_e<F16>(vr[i % A], pb[s], oacc[d]);
        if (i + A < N)
          vr[i % A] = tr_operand<C::BN>(vl, tl, 16 * ((i + A) / (D / 32)), 32 * ((i + A) % (D / 32)));
        __builtin_amdgcn_sched_barrier(0);
        if (s + 1 < NS) exps(s + 1, PPM * d, PPM * d + PPM);
        __builtin_amdgcn_sched_barrier(0);
      }
      l_i += ls;
    }
  };

  for (int kt = 0; kt < nkv; kt += 2) {
    step(kt, stage0, stage1);
    if (kt + 1 < nkv) step(kt + 1, stage1, stage0);
  }

  const float l_tot = wave_pair_sum(l_i);
  const float inv = 1.f / (l_tot + 1e-6f);
  if constexpr (D == 128) {
    // Epilogue: the ring is idle once every wave has left the loop, so each
    // wave stages its 32 rows of O there (wave w: stage w / 2, half w % 2)
    // and stores them as whole rows, 16 bytes per lane (a lane's own 8-byte
    // pieces of one row make every store instruction touch 32 partial lines:
    // c3's forward 90 -> 83 us).
    using OS = RowStage<D>;
    static_assert(2 * OS::BYTES <= C::STAGE, "the epilogue staging fits in a ring stage");
    __syncthreads();
    uint8_t* obuf = (wv < 2 ? stage0 : stage1) + (wv & 1) * OS::BYTES;
#pragma unroll
    for (int d = 0; d < D / 32; ++d)
#pragma unroll
      for (int g = 0; g < 4; ++g)
        OS::template put4<F16>(obuf, l32, d * 32 + 8 * g + 4 * hl, oacc[d][4 * g] * inv,
                 oacc[d][4 * g + 1] * inv, oacc[d][4 * g + 2] * inv, oacc[d][4 * g + 3] * inv);
    OS::store(obuf, seq_base<uint16_t>(P.o, p, b, e.q0, h) + (int64_t)wq0 * P.o.ss, P.o.ss,
              max(min(32, e.lq - wq0), 0), OS::CPR, lane);
  } else if (qvalid) {
    // (At d = 64 staging measured slower on the long dense tiles of c2 and
    // within noise elsewhere: the rows go out directly.)
    uint16_t* orow = seq_base<uint16_t>(P.o, p, b, e.q0, h) + (int64_t)qrow * P.o.ss;
#pragma unroll
    for (int d = 0; d < D / 32; ++d)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        u32x2 val;
        val[0] = pack_e<F16>(oacc[d][4 * g] * inv, oacc[d][4 * g + 1] * inv);
        val[1] = pack_e<F16>(oacc[d][4 * g + 2] * inv, oacc[d][4 * g + 3] * inv);
        *(u32x2*)(orow + d * 32 + 8 * g + 4 * hl) = val;
      }
  }
  if (qvalid && hl == 0) {
    float* lrow = seq_base<float>(P.lse, p, b, e.q0, h) + (int64_t)qrow * P.lse.ss;
    *lrow = (m_i == kNegInf)
                ? kNegInf
                : m_i * p.c + __builtin_amdgcn_logf(l_tot + 1e-6f) * kLn2;
  }
}

// One non-template kernel per (D, padded rank, element type): every kernel
// gets its own host launch stub.  WAVES: waves per SIMD the register budget
// is cut for.
#define FNA2_FWD_KERNEL(D, RNAME, RPL, S16, WAVES)                                          \
  __global__ __launch_bounds__(256, WAVES) void fwd_kernel_d##D##_r##RNAME(const FwdParams P) { \
    fwd_body<D, RPL, false, S16>(P);                                                         \
  }                                                                                          \
  __global__ __launch_bounds__(256, WAVES) void fwd_kernel_d##D##_r##RNAME##_f16(              \
      const FwdParams P) {                                                                   \
    fwd_body<D, RPL, true, S16>(P);                                                          \
  }
FNA2_FWD_KERNEL(64, 0, 0, false, 2)
FNA2_FWD_KERNEL(64, 16, 32, true, 2)
FNA2_FWD_KERNEL(64, 32, 32, false, 2)
FNA2_FWD_KERNEL(64, 64, 64, false, 2)
FNA2_FWD_KERNEL(128, 0, 0, false, 3)
FNA2_FWD_KERNEL(128, 32, 32, false, 3)
FNA2_FWD_KERNEL(128, 64, 64, false, 3)
#undef FNA2_FWD_KERNEL

}  // namespace

hipError_t launch_fwd(const FwdParams& P, int rpl, int grid, hipStream_t s) {
  if (grid <= 0) return hipSuccess;
  void (*k)(const FwdParams) = nullptr;
  // d = 64 with R <= 16: the split rank operand (S16)
  const bool r16 = rpl == 32 && P.p.R <= 16;
  if (P.p.f16) {
    if (P.p.D == 64)
      k = rpl == 0 ? fwd_kernel_d64_r0_f16
          : rpl == 32 ? (r16 ? fwd_kernel_d64_r16_f16 : fwd_kernel_d64_r32_f16)
                      : fwd_kernel_d64_r64_f16;
    if (P.p.D == 128)
      k = rpl == 0 ? fwd_kernel_d128_r0_f16 : rpl == 32 ? fwd_kernel_d128_r32_f16 : fwd_kernel_d128_r64_f16;
  } else {
    if (P.p.D == 64)
      k = rpl == 0 ? fwd_kernel_d64_r0
          : rpl == 32 ? (r16 ? fwd_kernel_d64_r16 : fwd_kernel_d64_r32) : fwd_kernel_d64_r64;
    if (P.p.D == 128) k = rpl == 0 ? fwd_kernel_d128_r0 : rpl == 32 ? fwd_kernel_d128_r32 : fwd_kernel_d128_r64;
  }
  if (!k || (rpl != 0 && rpl != 32 && rpl != 64)) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k, dim3(grid), dim3(256), 0, s, P);
  return hipGetLastError();
}

}  // namespace fna2
