// LDS tiles of 64 rows x DP bf16 for the gfx950 kernels: layout, staging and transposed reads.
//
// A tile is row-major (DP elements per row, no padding) with the 16-byte chunks of each row
// XOR-swizzled against bank conflicts: logical chunk c of row r sits at physical chunk
// c ^ tile_swz<DP>(r). For every read pattern of the kernels the swizzle value is a per-lane
// constant. The values were chosen by measurement (rocprofv3 SQ_LDS_BANK_CONFLICT): for DP = 96,
// bits 1-2 of the row, where bits 2-3 left the key kernel's LDS stalled on conflicts 18 % of its
// busy cycles and the forward's 10 % (bits 1-2: 1 % and 0.1 %, and a 9 % faster key kernel); for
// DP = 64, bits 0-2, where bits 1-3 left the forward 1.6 % and the key kernel 4.7 % (now 0.3 % and
// 2.7 %): a transposed read covers 8 rows x 2 chunks at once, and bits 0-2 give the four rows of
// each bank half distinct chunk pairs.
//
// Staging goes global -> LDS with global_load_lds_dwordx4: lane l of one wave instruction writes its
// 16 bytes at M0 + 16 l, so instruction n of a tile fills physical chunks 64 n .. 64 n + 63 and no
// registers carry the data.
//
// Transposed fragments come from ds_read_b64_tr_b16: within a 16-lane group, lane 4k+m pointing at
// row r0+k, columns [d0+4m, d0+4m+4) hands lane i the column d0+i of rows r0..r0+3.
#pragma once

#include <type_traits>
#include <utility>

#include "common.hpp"

namespace mote {

// f(integral_constant<int, 0>), ..., f(integral_constant<int, N - 1>): a loop whose index is a
// compile-time constant in every iteration.
template <typename F, int... I>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

// s_waitcnt immediate (gfx9 encoding) that waits until at most N vector-memory operations of the
// wave are outstanding, leaving the export and LDS/scalar counters unconstrained. Vector loads
// return in issue order, so after issuing stage A then stage B (N instructions), waiting for N
// leaves stage A complete.
template <int N>
__device__ constexpr int kVmWaitStage() {
  return (N & 0xF) | (0x7 << 4) | (0xF << 8) | (((N >> 4) & 0x3) << 14);
}

// Workgroup barrier of the staging loops. __syncthreads() carries a workgroup-scope release fence,
// which waits for every outstanding vector-memory operation of the wave, prefetches included; the
// loops instead wait for the stage they are about to read with kVmWaitStage and then need only
// their LDS operations complete before the barrier, so later stages stay in flight across it.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// One global -> LDS transfer of 16 bytes per active lane (lane l writes at l_base + 16 l, l_base
// wave-uniform), issued as inline assembly: the compiler does not track it, so it never adds a wait
// for it before unrelated LDS reads (its alias tracking of LDS DMA gives up at control-flow merges
// and then waits for every outstanding load, prefetches included). The kernels wait for each stage
// explicitly (kVmWaitStage, s_waitcnt 0); the compiler's own waits for register loads stay correct
// because vector-memory operations retire in issue order and it can only undercount younger ones.
__device__ __forceinline__ void lds_dma16(const void* g, void* l) {
  const uint32_t la = uint32_t(reinterpret_cast<uintptr_t>((void __attribute__((address_space(3)))*)l));
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(la) : "memory", "m0");
}

// The same with the SC1 cache-policy bit (agent scope): the data comes from the device-coherent
// level, not from a line of this XCD's L2 that another XCD's write-through stores left stale.
__device__ __forceinline__ void lds_dma16_sc1(const void* g, void* l) {
  const uint32_t la = uint32_t(reinterpret_cast<uintptr_t>((void __attribute__((address_space(3)))*)l));
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off sc1" ::"v"(g), "s"(la) : "memory", "m0");
}

// The same transfer from a wave-uniform base (SGPR pair) plus a per-lane byte offset. The offset
// registers can stay constant across a whole loop: a VMEM instruction reads its address registers
// only when the address unit takes it, so rewriting an address register right after an issue (the
// 64-bit form, one address per transfer) stalls the wave until the previous transfer has been taken.
__device__ __forceinline__ void lds_dma16_s(const void* base, uint32_t voff, void* l) {
  const uint32_t la = uint32_t(reinterpret_cast<uintptr_t>((void __attribute__((address_space(3)))*)l));
  asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(base), "s"(la) : "memory", "m0");
}

// The same with the LDS destination as a 32-bit LDS address, and no memory clobber: the transfer
// writes a stage slot that no instruction around it reads (the loops order slot reuse with their
// barriers, which do clobber memory), so the compiler may keep addresses and values in registers
// across it instead of reloading them after every transfer.
__device__ __forceinline__ void lds_dma16_sa(const void* base, uint32_t voff, uint32_t la) {
  asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(base), "s"(la) : "m0");
}
__device__ __forceinline__ uint32_t lds_addr(const void* l) {
  return uint32_t(reinterpret_cast<uintptr_t>((const void __attribute__((address_space(3)))*)l));
}

template <int DP>
__device__ __forceinline__ int tile_swz(int row) {
  if constexpr (DP == 64 || DP == 128) return row & 7;
  else return (row >> 1) & 3;  // DP 32 (4 chunks) and 96 (12 chunks): stays inside aligned groups of 4
}

typedef __attribute__((ext_vector_type(4))) short s16x4;

__device__ __forceinline__ bf16x4 lds_tr4(const bf16_t* p) {
  const s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((s16x4 __attribute__((address_space(3)))*)(p));
  return __builtin_bit_cast(bf16x4, v);
}

// Fragment (8 k-slots) of a transposed operand: lane (k4 = li / 4, m4 = li % 4) of group lg reads
// rows rb + 4 lg + k4 (slots 0..3) and rb + 16 + 4 lg + k4 (slots 4..7), columns 16 dt + 4 m4 ..
// +3, so lane li receives column 16 dt + li of rows rb + 4 lg .. +3 and rb + 16 + 4 lg .. +3 -- the
// permuted-k order {4g + r | 16 + 4g + r} of an accumulator pair.
template <int DP>
__device__ __forceinline__ typename Elem<bf16_t>::Frag tile_tr_frag(const bf16_t* tile, int rb, int dt, int li, int lg) {
  const int k4 = li >> 2, m4 = li & 3;
  const int c = 2 * dt + (m4 >> 1);
  const int r0 = rb + 4 * lg + k4, r1 = r0 + 16;
  const bf16x4 lo = lds_tr4(tile + r0 * DP + (c ^ tile_swz<DP>(r0)) * 8 + (m4 & 1) * 4);
  const bf16x4 hi = lds_tr4(tile + r1 * DP + (c ^ tile_swz<DP>(r1)) * 8 + (m4 & 1) * 4);
  typename Elem<bf16_t>::Frag f;
  f.v = bf16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  return f;
}

// Row fragment: row `row`, logical chunk `ch` (8 consecutive elements).
template <int DP>
__device__ __forceinline__ typename Elem<bf16_t>::Frag tile_row_frag(const bf16_t* tile, int row, int ch) {
  return Elem<bf16_t>::load8(tile + row * DP + (ch ^ tile_swz<DP>(row)) * 8);
}

// Staging of NT tiles per stage by the NW waves of a workgroup: the NT * CPR wave instructions are
// dealt round-robin over the waves; each lane precomputes, per instruction, the byte offset of its
// source chunk from the block's first row (row * stride + column), so a full block issues from a
// scalar base with constant offset registers. `wave` must be wave-uniform (readfirstlane), which
// keeps the LDS destinations and the per-block bases in scalar registers. Row strides must stay below
// 2^24 elements (checked by the host launchers), so the offsets fit 32 bits.
template <int DP, int NW, int NT>
struct TileStager {
  static constexpr int CPR = DP / 8;
  static constexpr int NINS = NT * CPR;
  static constexpr int PER = (NINS + NW - 1) / NW;
  uint32_t voff[PER];  // bytes

  __device__ __forceinline__ static int row_of(int n, int lane) { return (64 * n + lane) / CPR; }
  __device__ __forceinline__ static int col_of(int n, int lane) {
    const int q = 64 * n + lane;
    return ((q % CPR) ^ tile_swz<DP>(q / CPR)) * 8;
  }

  __device__ __forceinline__ void init(int wave, int lane, const int64_t (&stride)[NT]) {
    __builtin_assume(wave >= 0 && wave < NW);
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int ins = wave + NW * i;
      const int t = ins < NINS ? ins / CPR : 0, n = ins % CPR;
      voff[i] = uint32_t(row_of(n, lane) * int(stride[t]) + col_of(n, lane)) * 2u;
    }
  }

  // Rows r0 .. r0+63 of every source into dst, tiles back to back. Rows past rlast load a finite
  // copy of row rlast instead (the kernels mask them).
  __device__ __forceinline__ void issue(bf16_t* dst, const bf16_t* const (&src)[NT], const int64_t (&stride)[NT], int r0,
                                        int rlast, int wave, int lane) const {
    // the wave index is below NW: each transfer's tile t is then a constant of the unrolled loop
    __builtin_assume(wave >= 0 && wave < NW);
    if (__builtin_expect(r0 + 63 <= rlast, 1)) {
      // whole block in range: one scalar base per tile + the precomputed lane offsets
      const bf16_t* base[NT];
#pragma unroll
      for (int t = 0; t < NT; ++t) base[t] = src[t] + int64_t(r0) * stride[t];
      const uint32_t la = lds_addr(dst);
#pragma unroll
      for (int i = 0; i < PER; ++i) {
        const int ins = wave + NW * i;
        if (NINS % NW == 0 || ins < NINS) {
          const int t = ins / CPR, n = ins % CPR;
          lds_dma16_sa(base[t], voff[i], la + uint32_t(t * 64 * DP + n * 512) * 2u);
        }
      }
    } else {
      asm volatile("" ::: "memory");  // a separate path: keeps the full-block addresses free of clamping
#pragma unroll
      for (int i = 0; i < PER; ++i) {
        const int ins = wave + NW * i;
        if (NINS % NW == 0 || ins < NINS) {
          const int t = ins / CPR, n = ins % CPR;
          const int j = min(r0 + row_of(n, lane), rlast);
          load(src[t] + int64_t(j) * stride[t] + col_of(n, lane), dst + t * 64 * DP + n * 512);
        }
      }
    }
  }

  __device__ __forceinline__ static void load(const bf16_t* g, bf16_t* l) { lds_dma16(g, l); }
};

}  // namespace mote
