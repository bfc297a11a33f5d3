// fna2_tile.h — LDS tile machinery for the gfx950 kernels.
//
// Tiles are row-major in LDS (one row = one token, C 16-byte chunks of 8
// bf16) with the chunk index XOR-swizzled per row, so that both readers
// below are free of bank conflicts (checked for 32- and 64-bank LDS):
//   * row reads: ds_read_b128 by 32 lanes on 32 consecutive rows at the same
//     logical chunk (the natural MFMA operand, k = features);
//   * transpose reads: ds_read_b64_tr_b16 where each 16-lane group reads 4
//     consecutive rows x 4 consecutive chunks (an MFMA operand with k = rows).
// Tiles are filled by buffer_load ... lds (global -> LDS DMA, no VGPR
// staging).  A wave-level DMA instruction writes 64 consecutive 16-byte
// chunks; each lane fetches the logical chunk that belongs at its physical
// slot.  Rows beyond the tensor's valid range and chunks beyond the feature
// count are fetched from an out-of-range offset, which the buffer unit
// returns as zeros.
#pragma once

#include "fna2_device.h"

namespace fna2 {

typedef short v4i16 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(3))) v4i16 lds_v4i16;

constexpr uint32_t kRsrcWord3 = 0x00020000u;  // raw buffer, 32-bit data format
constexpr uint32_t kOOB = 0x80000000u;        // offset that is always out of range

// Buffer resource covering `nbytes` from `base`; reads past it return zero.
// Callers pass wave-uniform values; they are moved to scalar registers so the
// descriptor is an SGPR quad (a VGPR descriptor forces a waterfall loop).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t nbytes) {
  const uint64_t a = (uint64_t)base;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)a);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(a >> 32));
  void* ub = (void*)(((uint64_t)hi << 32) | lo);
  return __builtin_amdgcn_make_buffer_rsrc(ub, (short)0,
                                           (int)__builtin_amdgcn_readfirstlane(nbytes),
                                           (int)kRsrcWord3);
}

// Per-row chunk swizzle for rows of C chunks (C in {4, 8, 16}); depends on r % 16.
template <int C>
__device__ __forceinline__ int swz(int r) {
  const int x = r & 15;
  if constexpr (C == 4) return (x ^ (x >> 2)) & 3;
  else if constexpr (C == 8) return (x ^ (x >> 2) ^ ((x >> 1) << 2)) & 7;
  else return (x ^ (x << 2)) & 15;
}

// Byte offset of logical (row, chunk) inside a tile with C chunks per row.
template <int C>
__device__ __forceinline__ int tile_off(int row, int chunk) {
  return (row * C + (chunk ^ swz<C>(row))) * 16;
}

// DMA plan of a ROWS x C-chunk tile shared by NWAVE waves: wave-instruction i
// (covering physical chunks 64i..64i+63) belongs to wave i % NWAVE.
template <int ROWS, int C, int NWAVE>
struct Dma {
  static constexpr int N = ROWS * C / 64;              // instructions per tile
  static constexpr int PER_WAVE = (N + NWAVE - 1) / NWAVE;
  static_assert(ROWS * C % 64 == 0, "tile must be a whole number of 1 KB wave loads");

  uint32_t voff[PER_WAVE > 0 ? PER_WAVE : 1];

  // row_bytes: tensor row stride in bytes; valid_chunks: chunks with data
  // (features / 8); chunks past it read zeros.
  __device__ __forceinline__ void init(int wave, int lane, uint32_t row_bytes, int valid_chunks) {
#pragma unroll
    for (int j = 0; j < PER_WAVE; ++j) {
      const int i = wave + j * NWAVE;
      const int p = 64 * i + lane;
      const int row = p / C;
      const int col = (p % C) ^ swz<C>(row);
      voff[j] = (i < N && col < valid_chunks) ? (uint32_t)row * row_bytes + (uint32_t)col * 16u
                                              : kOOB;
    }
  }

  // Issue without a plan: the lane offsets are formed on the fly (for tiles
  // that are loaded rarely, where holding the offsets would cost registers).
  __device__ __forceinline__ static void issue_direct(__amdgpu_buffer_rsrc_t rs, uint8_t* lds,
                                                      int wave, int lane, uint32_t row_bytes,
                                                      int valid_chunks) {
#pragma unroll
    for (int j = 0; j < PER_WAVE; ++j) {
      const int i = wave + j * NWAVE;
      const int p = 64 * i + lane;
      const int row = p / C;
      const int col = (p % C) ^ swz<C>(row);
      const uint32_t off = col < valid_chunks ? (uint32_t)row * row_bytes + (uint32_t)col * 16u
                                              : kOOB;
      if (i < N)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void*)(lds + i * 1024), 16, off, 0, 0,
                                                 0);
    }
  }

  // Issue this wave's share of the tile into LDS at `lds` (tile base).
  __device__ __forceinline__ void issue(__amdgpu_buffer_rsrc_t rs, uint8_t* lds, int wave) const {
#pragma unroll
    for (int j = 0; j < PER_WAVE; ++j) {
      const int i = wave + j * NWAVE;
      if (i < N)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void*)(lds + i * 1024), 16, voff[j], 0,
                                                 0, 0);
    }
  }
};

// Row read: 8 bf16 of logical chunk `chunk` of row `row`.
template <int C>
__device__ __forceinline__ bf16x8 row_read(const uint8_t* tile, int row, int chunk) {
  return as_bf16x8(*(const u32x4*)(tile + tile_off<C>(row, chunk)));
}

// Per-lane constants of a transpose read (see tr_operand).
struct TrLane {
  int row;    // 4*(lane/32) + (lane%16)/4
  int chunk;  // 2*((lane/16)%2) + (lane%4)/2
  int byte;   // 8*(lane%2)
  __device__ __forceinline__ explicit TrLane(int lane)
      : row(4 * (lane >> 5) + ((lane & 15) >> 2)),
        chunk(2 * ((lane >> 4) & 1) + ((lane & 3) >> 1)),
        byte(8 * (lane & 1)) {}
};

// MFMA operand (32 x 16, lane % 32 <-> tile column m0 + lane % 32, k <-> 16
// tile rows k0..k0+15 in the permuted order of an accumulator-built operand:
// element e of lane-half h is row k0 + 8*(e/4) + 4*h + e%4) from a row-major
// tile with C chunks per row.  Two ds_read_b64_tr_b16.
template <int C>
__device__ __forceinline__ bf16x8 tr_operand(const uint8_t* tile, const TrLane& t, int k0, int m0) {
  const int c = (m0 >> 3) + t.chunk;
  const int r0 = k0 + t.row, r1 = k0 + 8 + t.row;
  const v4i16 a = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (lds_v4i16*)(tile + tile_off<C>(r0, c) + t.byte));
  const v4i16 b = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (lds_v4i16*)(tile + tile_off<C>(r1, c) + t.byte));
  typedef short v8i16 __attribute__((ext_vector_type(8)));
  const v8i16 ab = __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7);
  return __builtin_bit_cast(bf16x8, ab);
}

// Ring barrier: wait until at most N of this wave's vector-memory operations
// (tile DMA included) are in flight and its LDS reads are done, then barrier
// the workgroup.  Each wave waits for its own DMA before the barrier, so after
// it every wave's part of the older tiles is in LDS.  __syncthreads() is not
// used because its release fence waits for every in-flight LDS DMA (vmcnt(0))
// and so would drain the prefetch ring at each step.  The signal fences stop
// the compiler from moving memory accesses across the barrier.
template <int N>
__device__ __forceinline__ void ring_barrier() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4));  // lgkmcnt(0)
  __builtin_amdgcn_s_barrier();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

}  // namespace fna2
