// fna2_device.h — device-side types and helpers shared by the gfx950 kernels.
//
// Conventions used by every kernel in this directory:
//  * bf16 tensors are addressed as uint16_t; strides are in elements.
//  * The augmented contraction: for query head h the kernels form
//        S_ij / c = b_h * <Rq_i, Rk_j> + <a * Q_i, K_j>
//    as one MFMA accumulator: the rank chain first (bf16 products, exact in
//    fp32, fp32 sums), that accumulator scaled by b_h in fp32, then the
//    head-dim chain accumulated on top.  The host picks c > 0 and a in
//    {1,-1,0} with c * a = softmax_scale; b_h = graph_scale[h] / c.  No
//    operand is rounded beyond the bf16 inputs (a only flips or clears sign
//    bits), as in the reference, whose bias is an fp32 dot times graph_scale
//    in fp32 (FNA2/flash_naylis_attn.py:157-165).
//  * MFMA: v_mfma_f32_32x32x16_bf16.  Operand lane layout (A rows / B columns
//    on lane % 32, the 8 k-values of a 16-deep step on lane / 32) and the
//    accumulator layout (column = lane % 32, row = 8*(v/4) + 4*(lane/32) + v%4
//    for accumulator register v) are the CDNA 32x32 layouts.  A 16-deep step
//    built from accumulator registers 8s..8s+7 therefore holds rows
//    16s + perm16(8*(lane/32) + e), e = 0..7, with perm16 below; operands that
//    are read from LDS to meet such a register operand store their 16-row
//    groups in that permuted order.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>
#include <utility>

namespace fna2 {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kNegInf = -__builtin_inff();

// One tensor view: base + element strides (batch, sequence/token, head).
struct TView {
  const void* ptr;
  int64_t sb, ss, sh;
};

// Everything a kernel needs to know about the problem, passed by value.
struct Problem {
  int varlen;
  int nseq;        // dense B or varlen N
  int sq, sk;      // dense lengths (varlen: unused)
  int total_q, total_k;
  int H, H_KV, H_G, D, R;
  int causal;
  int f16;         // head-dim tensors are fp16 (else bf16); picks the kernel
  int group;       // H / H_KV
  float c;         // positive score multiplier
  float c2;        // c * log2(e)
  float qa;        // a in {1, -1, 0}
  const int* cu_q;
  const int* cu_k;
};

// Sequence extents, clamped so that no access leaves [0, total).
struct SeqExt {
  int q0, lq, k0, lk;
};

// f(std::integral_constant<int, i>) for i = 0 .. N-1, unrolled at compile
// time (for operands that must be immediates).
template <typename F, int... I>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

// Marks a value that is the same in every lane as wave-uniform (scalar).
__device__ __forceinline__ int uni(int x) { return __builtin_amdgcn_readfirstlane(x); }
__device__ __forceinline__ float uni_f(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, x)));
}

// A wave-uniform float, opaque to the compiler where it is used: `acc *=
// here_s(b)` for a 16-wide accumulator then multiplies by one scalar
// register, instead of a splat of b that the compiler hoists out of the
// loop and holds in 16 scalar registers (forcing other scalars to spill).
__device__ __forceinline__ float here_s(float x) {
  asm volatile("" : "+s"(x));
  return x;
}

// Extents of sequence b (b may differ per lane).
__device__ __forceinline__ SeqExt seq_ext(const Problem& p, int b) {
  SeqExt e;
  if (p.varlen) {
    int qs = p.cu_q[b], qe = p.cu_q[b + 1];
    int ks = p.cu_k[b], ke = p.cu_k[b + 1];
    qs = min(max(qs, 0), p.total_q);
    qe = min(max(qe, qs), p.total_q);
    ks = min(max(ks, 0), p.total_k);
    ke = min(max(ke, ks), p.total_k);
    e.q0 = qs; e.lq = qe - qs; e.k0 = ks; e.lk = ke - ks;
  } else {
    e.q0 = 0; e.lq = p.sq; e.k0 = 0; e.lk = p.sk;
  }
  return e;
}

// Read-only data that a kernel reads at wave-uniform addresses is read
// through the constant address space, so that the loads are scalar (s_load).
// A vector load there would be followed by a vmcnt wait, which also waits for
// every tile DMA in flight.
template <typename T>
__device__ __forceinline__ const __attribute__((address_space(4))) T* const_space(const T* ptr) {
  return (const __attribute__((address_space(4))) T*)ptr;
}

// Extents of a sequence b that is the same in every lane (scalar registers).
__device__ __forceinline__ SeqExt seq_ext_uniform(const Problem& p, int b) {
  SeqExt u;
  if (p.varlen) {
    const auto cq = const_space(p.cu_q);
    const auto ck = const_space(p.cu_k);
    b = uni(b);
    int qs = cq[b], qe = cq[b + 1];
    int ks = ck[b], ke = ck[b + 1];
    qs = min(max(qs, 0), p.total_q);
    qe = min(max(qe, qs), p.total_q);
    ks = min(max(ks, 0), p.total_k);
    ke = min(max(ke, ks), p.total_k);
    u.q0 = qs; u.lq = qe - qs; u.k0 = ks; u.lk = ke - ks;
  } else {
    u.q0 = 0; u.lq = p.sq; u.k0 = 0; u.lk = p.sk;
  }
  return u;
}

// A varlen work tile: sequence b, tile t within it and the sequence's clamped
// extents, so that a kernel decodes a tile with one 32-byte scalar load.
// slot: the tile's position in (sequence, tile) order, whatever order the
// list holds it in (sums over tiles index by it, so they do not depend on
// the list's order).
struct __attribute__((aligned(32))) TileRec {
  int b, t, q0, lq, k0, lk, slot, pad;
};

__device__ __forceinline__ int tile_slot(const TileRec* __restrict__ tiles, int tix) {
  return uni((const_space(tiles) + uni(tix))->slot);
}

__device__ __forceinline__ void tile_decode(const TileRec* __restrict__ tiles, int tix, int& b,
                                            int& t, SeqExt& e) {
  const auto r = const_space(tiles) + uni(tix);
  b = uni(r->b);
  t = uni(r->t);
  e.q0 = uni(r->q0);
  e.lq = uni(r->lq);
  e.k0 = uni(r->k0);
  e.lk = uni(r->lk);
}

// Base pointer of sequence b, head h of a view; row r is at base + r * ss.
template <typename T>
__device__ __forceinline__ T* seq_base(const TView& t, const Problem& p, int b,
                                       int start, int h) {
  int64_t off = p.varlen ? (int64_t)start * t.ss : (int64_t)b * t.sb;
  return (T*)t.ptr + off + (int64_t)h * t.sh;
}

__device__ __forceinline__ f32x16 mfma32(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// Element type of the head-dim tensors (q, k, v, out, dout, dq, dk, dv):
// bf16, or fp16 where a kernel is instantiated with F16.  R_q, R_k and their
// gradients are bf16 in both, as the reference asserts
// (FNA2/flash_naylis_attn.py:1419-1420): the rank chain of the augmented
// contraction always runs on the bf16 MFMA, the head-dim chain and the P / dS
// products on the one of the element type, accumulating into the same fp32
// registers.  Operands travel as 16-byte bit patterns typed bf16x8.
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

template <bool F16>
__device__ __forceinline__ f32x16 mfma_e(bf16x8 a, bf16x8 b, f32x16 c) {
  if constexpr (F16)
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) {
  return __builtin_bit_cast(bf16x8, v);
}

__device__ __forceinline__ u32x4 as_u32x4(bf16x8 v) {
  return __builtin_bit_cast(u32x4, v);
}

__device__ __forceinline__ u32x4 ld16(const void* p) {
  return *(const u32x4*)p;
}

__device__ __forceinline__ void st16(void* p, u32x4 v) { *(u32x4*)p = v; }

// Round two floats to bf16 (RNE) and pack: lo in bits 0..15.
__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
  f32x2 x = {lo, hi};
  bf16x2 y = __builtin_convertvector(x, bf16x2);
  return __builtin_bit_cast(uint32_t, y);
}

// Round two floats to the element type (RNE) and pack: lo in bits 0..15.
template <bool F16>
__device__ __forceinline__ uint32_t pack_e(float lo, float hi) {
  if constexpr (F16) {
    f32x2 x = {lo, hi};
    f16x2 y = __builtin_convertvector(x, f16x2);
    return __builtin_bit_cast(uint32_t, y);
  } else {
    return pack_bf16(lo, hi);
  }
}

// The two element-type values of a packed word, as floats.
template <bool F16>
__device__ __forceinline__ float elt_lo(uint32_t w) {
  if constexpr (F16)
    return (float)__builtin_bit_cast(f16x2, w)[0];
  else
    return __builtin_bit_cast(float, w << 16);
}
template <bool F16>
__device__ __forceinline__ float elt_hi(uint32_t w) {
  if constexpr (F16)
    return (float)__builtin_bit_cast(f16x2, w)[1];
  else
    return __builtin_bit_cast(float, w & 0xffff0000u);
}

__device__ __forceinline__ float bf16_lo(uint32_t w) {
  return __builtin_bit_cast(float, w << 16);
}
__device__ __forceinline__ float bf16_hi(uint32_t w) {
  return __builtin_bit_cast(float, w & 0xffff0000u);
}

// Position of row k (0..15) inside a permuted 16-row group (see header).
__device__ __forceinline__ int perm16(int k) {
  return (k & 3) | (((k >> 3) & 1) << 2) | (((k >> 2) & 1) << 3);
}

// Transpose helper: element e (0..7) of four 16-byte rows r0..r3, packed as
// four bf16 (row order) into 8 bytes.
__device__ __forceinline__ u32x2 gather4(const u32x4& r0, const u32x4& r1,
                                         const u32x4& r2, const u32x4& r3, int e) {
  const int w = e >> 1;
  u32x2 out;
  if (e & 1) {
    out[0] = (r0[w] >> 16) | (r1[w] & 0xffff0000u);
    out[1] = (r2[w] >> 16) | (r3[w] & 0xffff0000u);
  } else {
    out[0] = (r0[w] & 0xffffu) | (r1[w] << 16);
    out[1] = (r2[w] & 0xffffu) | (r3[w] << 16);
  }
  return out;
}

__device__ __forceinline__ float wave_pair_max(float x) {
  return fmaxf(x, __shfl_xor(x, 32));
}
__device__ __forceinline__ float wave_pair_sum(float x) {
  return x + __shfl_xor(x, 32);
}

__device__ __forceinline__ int cdiv(int a, int b) { return (a + b - 1) / b; }

}  // namespace fna2
