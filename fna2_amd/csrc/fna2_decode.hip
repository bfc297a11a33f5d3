// fna2_decode.hip — one-token decode against a KV cache for gfx950.
//
// Each sequence b has one new query row per head and a cache of len_b key /
// value rows (and, for the graph heads, Rk rows).  The score of query head h
// against cache row j is the attention score of the training kernels,
//     S_j = softmax_scale <q_h, K_j> + [h < H_G] graph_scale[h] <rq_h, Rk_hj>,
// with every row j < len_b visible.  This is row len_b - 1 of the causal
// forward over the whole sequence, so a model decodes with the bias it was
// trained with.  The reference decodes through PyTorch SDPA without the bias
// (FNA2/attention_fna2.py:412-429, :445-473), because it keeps no Rk for the
// cached rows.  With heads_graph = 0 this kernel computes exactly that
// reference decode.
//
// Work unit = (sequence, KV head, key split), one wave per unit.  The
// group's H / H_KV query heads are the 32 columns of the MFMA tile; unused
// columns hold zero queries.  Per 32-key step the wave forms
// S^T = Ka Qa^T as 32 keys x 32 head columns, with one MFMA chain over the
// augmented width D + (graph heads x R):
//   * Ka's rank part is the concatenation [Rk_h0 | Rk_h1 | ...] of the group's
//     graph heads;
//   * Qa's rank part is block diagonal: column i holds rq_h only in head
//     i's block;
// so each head gets its own bias from one contraction.  The rank chain runs
// first and its accumulator is scaled per column by graph_scale[h] / c in
// fp32 before the head-dim chain is added (no rounded operand).  The online
// softmax runs per column.  O^T += V^T P^T takes V^T from the row-major V tile
// through ds_read_b64_tr_b16, as in the forward kernel.
//
// K, Rk and V tiles are DMA'd global -> LDS (buffer_load ... lds) into a
// ring of NS stages private to the wave, NS - 1 tiles ahead of the compute.
// Rows past the split are zero-filled (K, V: descriptor bounds; Rk: an
// out-of-range offset) and their scores masked.  The path is bound by HBM
// (one pass over the cache), so the ring depth and the number of resident
// waves, not the MFMA count, set its speed.
//
// With several splits, each unit writes its unnormalised numerator and its
// (max, sum) pair to the workspace, and the merge kernel combines them into
//     O = sum_s e^{c (m_s - M)} acc_s / (sum_s e^{c (m_s - M)} l_s + 1e-6),
// the forward kernel's normalisation (FNA2/flash_naylis_attn.py:192-195).
#include "fna2_kernels.h"
#include "fna2_tile.h"

namespace fna2 {

namespace {

constexpr int kDecBN = 32;  // keys per step (one 32 x 32 MFMA block)

template <int D, int RC, int NS>
struct DecCfg {
  static constexpr int CD = D / 8;      // chunks per K / V row
  static constexpr int KSD = D / 16;    // 16-deep steps over the head dim
  static constexpr int KSR = RC / 2;    // ... over the concatenated rank chunks
  static constexpr int KBYTES = kDecBN * D * 2;
  static constexpr int RBYTES = kDecBN * RC * 16;
  static constexpr int STAGE = 2 * KBYTES + RBYTES;
  static constexpr int NRK = RC / 2;    // DMA instructions per Rk tile
  // VMEM instructions per step (a constant: the ring waits are immediates)
  static constexpr int OPS = 2 * (CD / 2) + NRK;
  static_assert(RC % 4 == 0, "rank chunks come in column groups of 4");
  static_assert(NS >= 2 && NS <= 4 && (NS - 2) * OPS < 64, "ring depth");
};

// Wait until at most N of this wave's vector-memory operations are in flight
// and its LDS reads are done.  The wave owns its ring, so no barrier.
template <int N>
__device__ __forceinline__ void wave_wait() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4));  // lgkmcnt(0)
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

template <int D, int RC, int NS>
__device__ __forceinline__ void decode_body(const DecodeParams& P) {
  using C = DecCfg<D, RC, NS>;
  // Stages as separate objects, so that the compiler can tell a DMA into one
  // from reads of another.
  __shared__ __attribute__((aligned(1024))) uint8_t st0[C::STAGE];
  __shared__ __attribute__((aligned(1024))) uint8_t st1[C::STAGE];
  __shared__ __attribute__((aligned(1024))) uint8_t st2[NS > 2 ? C::STAGE : 16];
  __shared__ __attribute__((aligned(1024))) uint8_t st3[NS > 3 ? C::STAGE : 16];
  const int lane = threadIdx.x;
  const int col = lane & 31, hl = lane >> 5;  // head column in the group; k half
  const int u = blockIdx.x;
  const int kvh = u % P.H_KV;
  const int b = (u / P.H_KV) % P.B;
  const int sp = u / (P.H_KV * P.B);
  int len = P.max_len;
  if (P.seqlens) len = min(max(uni(*const_space(P.seqlens + b)), 0), P.max_len);
  const int k_lo = sp * P.split_keys;
  const int k_hi = min(len, k_lo + P.split_keys);
  const int nt = k_hi > k_lo ? cdiv(k_hi - k_lo, kDecBN) : 0;
  const int h0 = kvh * P.group;
  const int gg = (RC > 0) ? min(max(P.H_G - h0, 0), P.group) : 0;  // graph heads here
  const int crr = P.R / 8;                                          // chunks per Rk row
  const int rch = gg * crr;                                         // rank chunks used
  const int nrs = cdiv(rch, 2);                                     // rank k-steps used

  const uint16_t* kb = (const uint16_t*)P.k.ptr + (int64_t)b * P.k.sb + (int64_t)kvh * P.k.sh;
  const uint16_t* vb = (const uint16_t*)P.v.ptr + (int64_t)b * P.v.sb + (int64_t)kvh * P.v.sh;
  const uint32_t krb = (uint32_t)P.k.ss * 2u, vrb = (uint32_t)P.v.ss * 2u;
  Dma<kDecBN, C::CD, 1> dk, dv;
  dk.init(0, lane, krb, C::CD);
  dv.init(0, lane, vrb, C::CD);

  // Rk tile: row = key, chunk c = graph head c / crr, chunk c % crr of its
  // row.  Wave instruction i fills rows 16 (i % 2) + lane / 4 of column
  // group i / 2.
  const uint16_t* rkb = kb;
  uint32_t roff[RC > 0 ? C::NRK : 1];
  if constexpr (RC > 0) {
    if (gg > 0) rkb = (const uint16_t*)P.rk.ptr + (int64_t)b * P.rk.sb + (int64_t)h0 * P.rk.sh;
    const uint32_t hs = (uint32_t)P.rk.sh * 2u, rs = (uint32_t)P.rk.ss * 2u;
#pragma unroll
    for (int i = 0; i < C::NRK; ++i) {
      const int row = 16 * (i & 1) + (lane >> 2);
      const int c = 4 * (i >> 1) + ((lane & 3) ^ swz4(row));
      roff[i] = c < rch ? (uint32_t)(c / crr) * hs + (uint32_t)row * rs + (uint32_t)(c % crr) * 16u
                        : kOOB;
    }
  }
  auto issue = [&](int t, uint8_t* base) {
    const int k0 = k_lo + t * kDecBN;
    const int rows = max(min(kDecBN, k_hi - k0), 0);  // 0 past the split: all zeros
    const int kr = min(k0, max(len - 1, 0));           // in-range base row
    dk.issue(make_rsrc(kb + (int64_t)kr * P.k.ss, (uint32_t)rows * krb), base, 0);
    if constexpr (RC > 0) {
      const auto rr = make_rsrc(rkb + (int64_t)kr * P.rk.ss, 0x7ffffff0u);
#pragma unroll
      for (int i = 0; i < C::NRK; ++i) {
        const int row = 16 * (i & 1) + (lane >> 2);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rr, (lds_void*)(base + C::KBYTES + i * 1024), 16,
                                                 row < rows ? roff[i] : kOOB, 0, 0, 0);
      }
    }
    dv.issue(make_rsrc(vb + (int64_t)kr * P.v.ss, (uint32_t)rows * vrb),
             base + C::KBYTES + C::RBYTES, 0);
  };
  auto stage = [&](auto si) -> uint8_t* {
    constexpr int s = decltype(si)::value;
    return s == 0 ? st0 : s == 1 ? st1 : s == 2 ? st2 : st3;
  };

  // The first NS - 1 tiles go out before the query loads, so the latencies
  // overlap.
  static_for<NS - 1>([&](auto si) { issue(decltype(si)::value, stage(si)); });
  __builtin_amdgcn_sched_barrier(0);

  // Query operand (B of S^T): lane holds Qa[col][16 s + 8 hl .. +7].
  bf16x8 qreg[C::KSD + (RC > 0 ? C::KSR : 0)];
  float bh = 0.f;  // graph_scale / c of this lane's head column (0: no bias)
  {
    const uint16_t* qb = (const uint16_t*)P.q.ptr + (int64_t)b * P.q.sb + (int64_t)h0 * P.q.sh;
    const auto rs = make_rsrc(qb, 0x7ffffff0u);
    const bool live = col < P.group;
    const uint32_t vo = (uint32_t)col * (uint32_t)P.q.sh * 2u + (uint32_t)(16 * hl);
    const uint32_t qxor = P.qa < 0.f ? 0x80008000u : 0u;
    const uint32_t qand = P.qa == 0.f ? 0u : 0xffffffffu;
#pragma unroll
    for (int s = 0; s < C::KSD; ++s) {
      u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rs, live ? vo + 32u * s : kOOB, 0, 0);
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = (v[i] & qand) ^ qxor;
      qreg[s] = as_bf16x8(v);
    }
    if constexpr (RC > 0) {
      const bool g = col < gg;
      const uint16_t* rqb = g ? (const uint16_t*)P.rq.ptr + (int64_t)b * P.rq.sb +
                                    (int64_t)h0 * P.rq.sh
                              : qb;
      const auto rr = make_rsrc(rqb, g ? 0x7ffffff0u : 0u);
      bh = g ? P.gs[h0 + col] / P.c : 0.f;
      const uint32_t ro = (uint32_t)col * (uint32_t)P.rq.sh * 2u;
#pragma unroll
      for (int s = 0; s < C::KSR; ++s) {
        const int c = 2 * s + hl;  // concatenated chunk of this lane
        const bool in = g && c < rch && c / crr == col;
        qreg[C::KSD + s] = as_bf16x8(__builtin_amdgcn_raw_buffer_load_b128(
            rr, in ? ro + (uint32_t)(c % crr) * 16u : kOOB, 0, 0));
      }
    }
  }

  f32x16 oacc[D / 32];
#pragma unroll
  for (int d = 0; d < D / 32; ++d) oacc[d] = f32x16{};
  float m_i = kNegInf, l_i = 0.f;
  const TrLane tl(lane);
  const RowLane rdl(lane);

  // One step: wait for tile t, refill the stage freed by step t - 1 with
  // tile t + NS - 1 (zeros past the split), compute on tile t.
  auto step = [&](int t, const uint8_t* cur, uint8_t* nxt) {
    wave_wait<(NS - 2) * C::OPS>();
    issue(t + NS - 1, nxt);
    __builtin_amdgcn_sched_barrier(0);
    const uint8_t* kl = cur;
    const uint8_t* rl = kl + C::KBYTES;
    const uint8_t* vl = rl + C::RBYTES;
    // S^T / c: the rank chain (block-diagonal Rq: each column sees only its
    // own head's Rk chunks) scaled per column by that head's b in fp32, then
    // the head-dim chain on top.
    f32x16 acc = f32x16{};
    if constexpr (RC > 0) {
#pragma unroll
      for (int s = 0; s < C::KSR; ++s)
        if (s < nrs) acc = mfma32(row_read<kDecBN>(rl, rdl, 0, s), qreg[C::KSD + s], acc);
      acc *= bh;
    }
#pragma unroll
    for (int s = 0; s < C::KSD; ++s) acc = mfma32(row_read<kDecBN>(kl, rdl, 0, s), qreg[s], acc);
    const int kbase = k_lo + t * kDecBN;
    if (kbase + kDecBN > k_hi) {
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int key = kbase + 8 * (v >> 2) + 4 * hl + (v & 3);
        acc[v] = key >= k_hi ? kNegInf : acc[v];
      }
    }
    float mx = kNegInf;
#pragma unroll
    for (int v = 0; v < 16; ++v) mx = fmaxf(mx, acc[v]);
    mx = wave_pair_max(mx);
    const float m_new = fmaxf(m_i, mx);
    const float m_use = (m_new == kNegInf) ? 0.f : m_new;
    const float nm = -m_use * P.c2;
    float ls = 0.f;
    bf16x8 pb[2];
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      u32x4 pk;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int v0 = 8 * half + 2 * i;
        const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(acc[v0], P.c2, nm));
        const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(acc[v0 + 1], P.c2, nm));
        ls += p0 + p1;
        pk[i] = pack_bf16(p0, p1);
      }
      pb[half] = as_bf16x8(pk);
    }
    // The running maximum rarely moves once a few hundred keys are in: skip
    // the rescale when no column's maximum changed.
    if (__builtin_amdgcn_ballot_w64(m_new != m_i) != 0) {
      const float alpha = __builtin_amdgcn_exp2f((m_i - m_use) * P.c2);
      l_i *= alpha;
#pragma unroll
      for (int d = 0; d < D / 32; ++d) oacc[d] *= alpha;
    }
    l_i += ls;
    m_i = m_new;
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int d = 0; d < D / 32; ++d)
        oacc[d] = mfma32(tr_operand<kDecBN>(vl, tl, 16 * s, 32 * d), pb[s], oacc[d]);
  };

  for (int t = 0; t < nt; t += NS) {
    static_for<NS>([&](auto si) {
      constexpr int s = decltype(si)::value;
      if (t + s < nt) step(t + s, stage(si), stage(std::integral_constant<int, (s + NS - 1) % NS>{}));
    });
  }
  // Drain the ring: no DMA may still write into LDS when the wave ends.
  wave_wait<0>();

  const float l_tot = wave_pair_sum(l_i);
  if (col >= P.group) return;
  const int h = h0 + col;
  if (P.nsplit == 1) {
    const float inv = 1.f / (l_tot + 1e-6f);
    uint16_t* orow = (uint16_t*)P.o.ptr + (int64_t)b * P.o.sb + (int64_t)h * P.o.sh;
#pragma unroll
    for (int d = 0; d < D / 32; ++d)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        u32x2 val;
        val[0] = pack_bf16(oacc[d][4 * g] * inv, oacc[d][4 * g + 1] * inv);
        val[1] = pack_bf16(oacc[d][4 * g + 2] * inv, oacc[d][4 * g + 3] * inv);
        *(u32x2*)(orow + d * 32 + 8 * g + 4 * hl) = val;
      }
    if (hl == 0 && P.lse.ptr) {
      float* lrow = (float*)P.lse.ptr + (int64_t)b * P.lse.sb + (int64_t)h * P.lse.sh;
      *lrow = (m_i == kNegInf) ? kNegInf
                               : m_i * P.c + __builtin_amdgcn_logf(l_tot + 1e-6f) * kLn2;
    }
    return;
  }
  const int64_t row = ((int64_t)sp * P.B + b) * P.H + h;
  float* arow = P.acc + row * D;
#pragma unroll
  for (int d = 0; d < D / 32; ++d)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      f32x4_t val = {oacc[d][4 * g], oacc[d][4 * g + 1], oacc[d][4 * g + 2], oacc[d][4 * g + 3]};
      *(f32x4_t*)(arow + d * 32 + 8 * g + 4 * hl) = val;
    }
  if (hl == 0) *(f32x2*)(P.ml + 2 * row) = f32x2{m_i, l_tot};
}

// One wave per (sequence, head): combine the splits' partial results.
template <int D>
__device__ __forceinline__ void merge_body(const DecodeParams& P) {
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);  // b * H + h
  if (r >= (int64_t)P.B * P.H) return;
  const int b = (int)(r / P.H), h = (int)(r % P.H);
  const int64_t plane = (int64_t)P.B * P.H;  // rows per split
  float m = kNegInf, l = 0.f;
  if (lane < P.nsplit) {
    const f32x2 ml = *(const f32x2*)(P.ml + 2 * (lane * plane + r));
    m = ml[0];
    l = ml[1];
  }
  float M = m;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) M = fmaxf(M, __shfl_xor(M, off));
  const float w = (m == kNegInf) ? 0.f : __builtin_amdgcn_exp2f((m - M) * P.c2);
  float L = l * w;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) L += __shfl_xor(L, off);
  constexpr int E = D / 64;  // features per lane
  float o[E];
#pragma unroll
  for (int e = 0; e < E; ++e) o[e] = 0.f;
  for (int s = 0; s < P.nsplit; ++s) {
    const float ws = __shfl(w, s);
    const float* a = P.acc + (s * plane + r) * D + lane * E;
    if constexpr (E == 2) {
      const f32x2 x = *(const f32x2*)a;
      o[0] += ws * x[0];
      o[1] += ws * x[1];
    } else {
#pragma unroll
      for (int e = 0; e < E; ++e) o[e] += ws * a[e];
    }
  }
  const float inv = 1.f / (L + 1e-6f);
  uint16_t* orow = (uint16_t*)P.o.ptr + (int64_t)b * P.o.sb + (int64_t)h * P.o.sh + lane * E;
  if constexpr (E == 2) {
    *(uint32_t*)orow = pack_bf16(o[0] * inv, o[1] * inv);
  } else {
    orow[0] = (uint16_t)(pack_bf16(o[0] * inv, 0.f) & 0xffffu);
  }
  if (lane == 0 && P.lse.ptr) {
    float* lrow = (float*)P.lse.ptr + (int64_t)b * P.lse.sb + (int64_t)h * P.lse.sh;
    *lrow = (M == kNegInf) ? kNegInf : M * P.c + __builtin_amdgcn_logf(L + 1e-6f) * kLn2;
  }
}

#define FNA2_DEC_KERNEL(D, RC, NS)                                                        \
  __global__ __launch_bounds__(64, 1) void decode_kernel_d##D##_c##RC(const DecodeParams P) { \
    decode_body<D, RC, NS>(P);                                                          \
  }
FNA2_DEC_KERNEL(64, 0, kDecodeStages)
FNA2_DEC_KERNEL(64, 4, kDecodeStages)
FNA2_DEC_KERNEL(64, 8, kDecodeStages)
FNA2_DEC_KERNEL(64, 16, kDecodeStages)
FNA2_DEC_KERNEL(64, 32, kDecodeStages)
FNA2_DEC_KERNEL(128, 0, kDecodeStages)
FNA2_DEC_KERNEL(128, 4, kDecodeStages)
FNA2_DEC_KERNEL(128, 8, kDecodeStages)
FNA2_DEC_KERNEL(128, 16, kDecodeStages)
FNA2_DEC_KERNEL(128, 32, kDecodeStages)
#undef FNA2_DEC_KERNEL

__global__ __launch_bounds__(256) void decode_merge_d64(const DecodeParams P) { merge_body<64>(P); }
__global__ __launch_bounds__(256) void decode_merge_d128(const DecodeParams P) { merge_body<128>(P); }

}  // namespace

int decode_rank_chunks(int rch) {
  return rch <= 0 ? 0 : rch <= 4 ? 4 : rch <= 8 ? 8 : rch <= 16 ? 16 : rch <= 32 ? 32 : -1;
}

int decode_stage_bytes(int D, int rc) { return kDecBN * (2 * D * 2 + rc * 16); }

hipError_t launch_decode(const DecodeParams& P, int rc, hipStream_t s) {
  const int64_t units = (int64_t)P.B * P.H_KV * P.nsplit;
  if (units <= 0) return hipSuccess;
  void (*k)(const DecodeParams) = nullptr;
  if (P.D == 64)
    k = rc == 0 ? decode_kernel_d64_c0 : rc == 4 ? decode_kernel_d64_c4 : rc == 8 ? decode_kernel_d64_c8
      : rc == 16 ? decode_kernel_d64_c16 : rc == 32 ? decode_kernel_d64_c32 : nullptr;
  if (P.D == 128)
    k = rc == 0 ? decode_kernel_d128_c0 : rc == 4 ? decode_kernel_d128_c4 : rc == 8 ? decode_kernel_d128_c8
      : rc == 16 ? decode_kernel_d128_c16 : rc == 32 ? decode_kernel_d128_c32 : nullptr;
  if (!k) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k, dim3((uint32_t)units), dim3(64), 0, s, P);
  return hipGetLastError();
}

hipError_t launch_decode_merge(const DecodeParams& P, hipStream_t s) {
  const int64_t rows = (int64_t)P.B * P.H;
  if (rows <= 0 || P.nsplit <= 1) return hipSuccess;
  void (*k)(const DecodeParams) = P.D == 64 ? decode_merge_d64 : P.D == 128 ? decode_merge_d128 : nullptr;
  if (!k) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k, dim3((uint32_t)((rows + 3) / 4)), dim3(256), 0, s, P);
  return hipGetLastError();
}

}  // namespace fna2
