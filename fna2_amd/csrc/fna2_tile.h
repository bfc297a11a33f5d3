// fna2_tile.h — LDS tile machinery for the gfx950 kernels.
//
// A tile holds ROWS rows (one row = one token) of C 16-byte chunks (8 bf16
// each), C a multiple of 4.  The row is split into column groups of 4 chunks
// (32 features); group g is a ROWS x 64-byte sub-tile, and inside a row the
// 4 chunks of a group are XOR-swizzled by a 2-bit function of row bits 1..3:
//   offset(row, chunk) = (chunk / 4) * ROWS * 64 + row * 64
//                        + ((chunk % 4) ^ swz4(row)) * 16.
// Both readers below are free of bank conflicts with 32 and with 64 banks:
//   * row reads: ds_read_b128 by 32 lanes on 32 consecutive rows at the same
//     logical chunk (the natural MFMA operand, k = features);
//   * transpose reads: ds_read_b64_tr_b16 where each 16-lane group reads 4
//     consecutive rows x 2 consecutive chunks (an MFMA operand with k = rows).
// Because the swizzle only permutes chunks inside a group and only depends on
// row bits 1..3, moving a read by a multiple of 16 rows or by whole column
// groups moves its address by a constant: a lane needs two offsets for all
// its row reads of a tile and two for all its transpose reads, and every
// other term is an instruction immediate.
// Tiles are filled by buffer_load ... lds (global -> LDS DMA, no VGPR
// staging).  A wave-level DMA instruction writes 64 consecutive 16-byte
// slots; each lane fetches the logical chunk that belongs at its slot.  Rows
// beyond the tensor's valid range and chunks beyond the feature count are
// fetched from an out-of-range offset, which the buffer unit returns as zeros.
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

// Buffer descriptor as four scalar words, for inline assembly.
__device__ __forceinline__ u32x4 rsrc_words(const void* base, uint32_t nbytes) {
  const uint64_t a = (uint64_t)base;
  u32x4 w;
  w[0] = __builtin_amdgcn_readfirstlane((uint32_t)a);
  w[1] = __builtin_amdgcn_readfirstlane((uint32_t)(a >> 32)) & 0xffffu;
  w[2] = __builtin_amdgcn_readfirstlane(nbytes);
  w[3] = kRsrcWord3;
  return w;
}

// LDS byte address of a pointer into shared memory.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// Loads the compiler does not see as loads (inline assembly).  It therefore
// inserts no wait for them, neither before a use of the destination nor
// before an LDS read it cannot prove disjoint from an LDS DMA: every wait on
// them is the caller's, explicit.  Nor does its hazard recognizer see the
// buffer instruction: a VALU write of an SGPR (v_readfirstlane of a
// descriptor word) needs 5 wait states before a VMEM instruction reads it,
// so each block starts with s_nop 4.
//   dma_lds<16|4>: global -> LDS DMA of 16 (4) bytes per lane to lds + 16
//     (4) * lane, from byte voffset of the buffer.
//   load16_inplace<IMM>: 16 bytes at voffset + IMM into the registers that
//     hold `dst` (which the caller must not read before its wait).
// (The DMA takes its LDS address from M0, which it clobbers: nothing else
// in these kernels keeps a value in M0.)
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
template <int BYTES>
__device__ __forceinline__ void dma_lds(const u32x4& rs, uint32_t lds, uint32_t voffset) {
  static_assert(BYTES == 16 || BYTES == 4, "dword or dwordx4");
  if constexpr (BYTES == 16)
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 4\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
                 :
                 : "s"(lds), "v"(voffset), "s"(rs)
                 : "memory", "m0");
  else
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 4\n\tbuffer_load_dword %1, %2, 0 offen lds"
                 :
                 : "s"(lds), "v"(voffset), "s"(rs)
                 : "memory", "m0");
}
#pragma clang diagnostic pop
template <int IMM>
__device__ __forceinline__ void load16_inplace(u32x4& dst, const u32x4& rs, uint32_t voffset) {
  static_assert(IMM >= 0 && IMM < 4096, "buffer offset field");
  asm volatile("s_nop 4\n\tbuffer_load_dwordx4 %0, %1, %2, 0 offen offset:%3"
               : "+v"(dst)
               : "v"(voffset), "s"(rs), "i"(IMM));
}

// 16-byte LDS read at byte address lds + IMM into the registers that hold
// `dst`, in place (the caller waits: lgkmcnt).
template <int IMM>
__device__ __forceinline__ void ds_read16_inplace(u32x4& dst, uint32_t lds) {
  static_assert(IMM >= 0 && IMM < 65536, "ds offset field");
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "+v"(dst) : "v"(lds), "i"(IMM));
}

// 2-bit chunk swizzle of a row (row bits 1..3).
__device__ __forceinline__ int swz4(int r) {
  return ((((r >> 1) ^ (r >> 3)) & 1) << 1) | ((r >> 2) & 1);
}

// Byte offset of logical (row, chunk) inside a tile of ROWS rows.
template <int ROWS>
__device__ __forceinline__ int tile_off(int row, int chunk) {
  return (chunk >> 2) * (ROWS * 64) + row * 64 + (((chunk & 3) ^ swz4(row)) << 4);
}

// DMA plan of a ROWS x C-chunk tile shared by NWAVE waves: wave-instruction i
// (covering physical chunks 64i..64i+63) belongs to wave i % NWAVE.
template <int ROWS, int C, int NWAVE>
struct Dma {
  static constexpr int N = ROWS * C / 64;              // instructions per tile
  static constexpr int PER_WAVE = (N + NWAVE - 1) / NWAVE;
  static_assert(ROWS * C % 64 == 0, "tile must be a whole number of 1 KB wave loads");
  static_assert(C % 4 == 0 && ROWS % 16 == 0, "tile shape");

  uint32_t voff[PER_WAVE > 0 ? PER_WAVE : 1];

  // row_bytes: tensor row stride in bytes; valid_chunks: chunks with data
  // (features / 8); chunks past it read zeros.
  __device__ __forceinline__ void init(int wave, int lane, uint32_t row_bytes, int valid_chunks,
                                       bool mirror = false) {
#pragma unroll
    for (int j = 0; j < PER_WAVE; ++j)
      voff[j] = slot_offset(wave + j * NWAVE, lane, row_bytes, valid_chunks, mirror);
  }

  // Global byte offset of the chunk that lands in slot 64 i + lane.  With
  // `mirror` (a 4-chunk row holding at most 2 chunks of data), chunks 2 and
  // 3 load the data of chunks 0 and 1 again.
  __device__ __forceinline__ static uint32_t slot_offset(int i, int lane, uint32_t row_bytes,
                                                         int valid_chunks, bool mirror = false) {
    const int p = 64 * i + lane;
    const int grp = p / (ROWS * 4);
    const int rem = p - grp * (ROWS * 4);
    const int row = rem >> 2;
    int col = 4 * grp + ((rem & 3) ^ swz4(row));
    if (mirror) col &= 1;
    return (i < N && col < valid_chunks) ? (uint32_t)row * row_bytes + (uint32_t)col * 16u : kOOB;
  }

  // Issue without a plan: the lane offsets are formed on the fly (for tiles
  // that are loaded rarely, where holding the offsets would cost registers).
  __device__ __forceinline__ static void issue_direct(__amdgpu_buffer_rsrc_t rs, uint8_t* lds,
                                                      int wave, int lane, uint32_t row_bytes,
                                                      int valid_chunks) {
#pragma unroll
    for (int j = 0; j < PER_WAVE; ++j) {
      const int i = wave + j * NWAVE;
      if (i < N)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            rs, (lds_void*)(lds + i * 1024), 16, slot_offset(i, lane, row_bytes, valid_chunks), 0,
            0, 0);
    }
  }

  // Issue exactly PER_WAVE instructions, whatever the wave: a share past
  // the tile repeats share i % N (the same bytes to the same place, so the
  // two writes agree).  The count of VMEM instructions is then a constant,
  // which lets waits on the DMA ring be instruction immediates, and every
  // destination lies in the tile (no select between LDS objects, which
  // would defeat the compiler's alias analysis of DMA against LDS reads).
  // Needs init_fixed.
  __device__ __forceinline__ void init_fixed(int wave, int lane, uint32_t row_bytes,
                                             int valid_chunks) {
#pragma unroll
    for (int j = 0; j < PER_WAVE; ++j)
      voff[j] = slot_offset((wave + j * NWAVE) % N, lane, row_bytes, valid_chunks);
  }
  __device__ __forceinline__ void issue_fixed(const u32x4& rs, uint8_t* lds, int wave,
                                              uint32_t add) const {
#pragma unroll
    for (int j = 0; j < PER_WAVE; ++j) {
      const int i = (wave + j * NWAVE) % N;
      dma_lds<16>(rs, lds_addr(lds + i * 1024), voff[j] + add);
    }
  }

  // Issue this wave's share of a tile whose first row is `add` bytes past
  // the descriptor's base (out-of-range lane offsets stay out of range as
  // long as add < 2^31).
  __device__ __forceinline__ void issue_at(__amdgpu_buffer_rsrc_t rs, uint8_t* lds, int wave,
                                           uint32_t add) const {
#pragma unroll
    for (int j = 0; j < PER_WAVE; ++j) {
      const int i = wave + j * NWAVE;
      if (i < N)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void*)(lds + i * 1024), 16,
                                                 voff[j] + add, 0, 0, 0);
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

// Per-lane offsets of row reads: lane reads row r0 + lane % 32 (r0 a
// multiple of 16) at chunk 2s + lane / 32, the A operand of k-step s.
struct RowLane {
  int off[2];  // for even and odd s
  __device__ __forceinline__ explicit RowLane(int lane) {
    const int l = lane & 31, hl = lane >> 5;
#pragma unroll
    for (int j = 0; j < 2; ++j) off[j] = l * 64 + (((2 * j + hl) ^ swz4(l)) << 4);
  }
};

// Row read: 8 bf16 of chunk 2s + lane / 32 of row r0 + lane % 32.
template <int ROWS>
__device__ __forceinline__ bf16x8 row_read(const uint8_t* tile, const RowLane& t, int r0, int s) {
  return as_bf16x8(*(const u32x4*)(tile + (s >> 1) * (ROWS * 64) + r0 * 64 + t.off[s & 1]));
}

// Per-lane offsets of a transpose read: lane % 16 / 4 and lane / 32 pick the
// row (0..7), (lane / 16) % 2 and lane % 4 / 2 the chunk in a column group,
// lane % 2 the 8-byte half; the second read is 8 rows further down.
struct TrLane {
  int off0, off1;
  __device__ __forceinline__ explicit TrLane(int lane) {
    const int row = 4 * (lane >> 5) + ((lane & 15) >> 2);
    const int chunk = 2 * ((lane >> 4) & 1) + ((lane & 3) >> 1);
    const int byte = 8 * (lane & 1);
    off0 = row * 64 + ((chunk ^ swz4(row)) << 4) + byte;
    off1 = (row + 8) * 64 + ((chunk ^ swz4(row + 8)) << 4) + byte;
  }
};

// MFMA operand (32 x 16, lane % 32 <-> tile column m0 + lane % 32, k <-> 16
// tile rows k0..k0+15 in the permuted order of an accumulator-built operand:
// element e of lane-half h is row k0 + 8*(e/4) + 4*h + e%4) from a tile of
// ROWS rows; k0 a multiple of 16, m0 of 32.  Two ds_read_b64_tr_b16.
template <int ROWS>
__device__ __forceinline__ bf16x8 tr_operand(const uint8_t* tile, const TrLane& t, int k0, int m0) {
  const uint8_t* base = tile + (m0 >> 5) * (ROWS * 64) + k0 * 64;
  const v4i16 a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(base + t.off0));
  const v4i16 b = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(base + t.off1));
  typedef short v8i16 __attribute__((ext_vector_type(8)));
  const v8i16 ab = __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7);
  return __builtin_bit_cast(bf16x8, ab);
}

// Epilogue staging of a wave's 32 output rows of W 16-bit values (W = 32,
// 64 or 128) in LDS, so that global stores write whole rows.  The accumulators
// hold, per lane, 4 consecutive values of one row (row = lane % 32), so a
// staging write is an 8-byte write by 32 rows x 2 halves of one 16-byte
// chunk, and a store reads whole chunks (ds_read_b128) of RPI rows.  Row r
// sits at r * 2W bytes; its chunk c sits in 16-byte slot pos(r, c) (a
// permutation of the row's slots), with its two 8-byte halves exchanged
// when hswap(r) = 1.  The 32 rows of a write then cover 32 distinct (slot,
// half) pairs, so every 8-byte write and every 16-byte read is free of bank
// conflicts with 32 banks (16 lanes of a b64 / 8 of a b128 access per
// cycle) and with 64 banks (32 / 16 lanes per cycle).  (A plain chunk
// rotation by row, with no half exchange, leaves rows r and r + 16 of a
// write on the same banks.)  For W = 128 and 64, hswap depends on row bits
// 3 and 4 only, which a store's lane never sets, so the exchange on reading
// is a register renaming; for W = 32 it is a per-lane select.
template <int W>
struct RowStage {
  static constexpr int CPR = W / 8;              // 16-byte chunks per row
  static constexpr int RPI = 64 / CPR;           // rows per wave-wide 16-byte access
  static constexpr int BYTES = 32 * W * 2;       // one wave's rows
  static_assert(W == 32 || W == 64 || W == 128, "row width");
  __device__ __forceinline__ static int pos(int r, int c) {
    if constexpr (W == 128) return c ^ (r & 15);
    else if constexpr (W == 64) return c ^ (((r >> 1) & 3) | (((r ^ (r >> 3)) & 1) << 2));
    else return c ^ ((r >> 2) & 3);
  }
  __device__ __forceinline__ static int hswap(int r) {
    if constexpr (W == 32) return ((r >> 1) ^ (r >> 4)) & 1;
    else return ((r >> 3) ^ (r >> 4)) & 1;
  }
  // Byte offset of values col .. col + 3 (col a multiple of 4) of row `row`.
  __device__ __forceinline__ static int off(int row, int col) {
    return row * W * 2 + (pos(row, col >> 3) << 4) + ((((col >> 2) & 1) ^ hswap(row)) << 3);
  }
  // 4 values (col a multiple of 4) of row `row`, rounded to bf16 (fp16
  // with F16).
  template <bool F16 = false>
  __device__ __forceinline__ static void put4(uint8_t* buf, int row, int col, float a, float b,
                                              float c, float d) {
    u32x2 v;
    v[0] = pack_e<F16>(a, b);
    v[1] = pack_e<F16>(c, d);
    *(u32x2*)(buf + off(row, col)) = v;
  }
  // Stores rows [0, nrows) to dst + row * stride (elements), chunks [0,
  // valid_chunks) of each: RPI rows per wave-wide access.
  __device__ __forceinline__ static void store(const uint8_t* buf, uint16_t* dst, int64_t stride,
                                               int nrows, int valid_chunks, int lane) {
#pragma unroll
    for (int i = 0; i < 32 / RPI; ++i) {
      const int r = i * RPI + lane / CPR, ch = lane % CPR;
      const u32x4 s = *(const u32x4*)(buf + r * W * 2 + (pos(r, ch) << 4));
      const bool x = W == 32 ? hswap(r) != 0 : hswap(i * RPI) != 0;
      const u32x4 v = x ? u32x4{s[2], s[3], s[0], s[1]} : s;
      if (r < nrows && ch < valid_chunks) st16(dst + (int64_t)r * stride + ch * 8, v);
    }
  }
};

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
