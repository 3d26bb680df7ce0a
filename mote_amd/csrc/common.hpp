// Shared device helpers for the Relation kernels (gfx950 / CDNA4 only).
//
// Matrix products use the 16x16 MFMA family with one fragment convention for both element types:
// a fragment is 8 values per lane covering a 16 x 32 (rows x k) operand block, lane l holding row
// (l % 16) and the 8 k-slots of group (l / 16). bf16 blocks are one v_mfma_f32_16x16x32_bf16;
// fp32 blocks are eight v_mfma_f32_16x16x4_f32, slot j of every lane feeding the j-th instruction.
// Any assignment of k to (group, slot) is valid as long as the A and B fragments of one product use
// the same one, which lets the kernels feed the accumulator layout of one product straight into the
// next as a permuted-k operand.
//
// Accumulator (C) layout of a 16 x 16 tile: lane l holds rows 4*(l/16) + r, r = 0..3, of column l % 16.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

// Timestamp hook of the tile kernels' block loops: MOTE_STAMP(slot, iteration) marks the points
// (0 loop top, 1 after the prefetch issue, 2 after the block math, 3 after the load wait, 4 after the
// barrier). It compiles to nothing unless a profiling translation unit defines it before including a
// kernel source.
#ifndef MOTE_STAMP
#define MOTE_STAMP(slot, it) ((void)0)
#endif

namespace mote {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(4))) __bf16 bf16x4;
typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef uint16_t bf16_t;  // storage type of bf16 tensors (raw bits)

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kRescale = 8.0f;  // log2 units of slack before the online softmax rescales
constexpr float kNegInf = -__builtin_inff();

__device__ __forceinline__ float bf2f(bf16_t v) { return __uint_as_float(uint32_t(v) << 16); }
__device__ __forceinline__ bf16_t f2bf(float v) {
  __bf16 b = (__bf16)v;  // v_cvt_pk_bf16_f32: round to nearest even
  return __builtin_bit_cast(bf16_t, b);
}

// Fast hardware transcendentals (v_exp_f32 / v_rcp_f32, ~1 ulp) for the inner loops.
__device__ __forceinline__ float fexp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float frcp(float x) { return __builtin_amdgcn_rcpf(x); }
// Accurate sigmoid for the per-row epilogues.
__device__ __forceinline__ float sigmoid_acc(float x) { return 1.0f / (1.0f + expf(-x)); }

__device__ __forceinline__ float wave_xor(float v, int mask) { return __shfl_xor(v, mask, 64); }

// Max / sum over the four lanes li, li + 16, li + 32, li + 48 (one value per accumulator column)
// with the gfx950 row swaps: v_permlane16_swap / v_permlane32_swap of a register with itself put
// the partner row's value in one of the two results and the lane's own value in the other.
typedef __attribute__((ext_vector_type(2))) unsigned int u32x2;
// The max of two lanes' values without fmaxf's canonicalisation: the operands come back from the swap
// as integers, so the compiler quiets each one (a v_max of the value with itself) before the max. The
// inputs here are MFMA dot products or -inf, never signalling NaNs.
__device__ __forceinline__ float vmax_raw(float a, float b) {
  float r;
  asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
  return r;
}
__device__ __forceinline__ float lanegroup_max(float x) {
  const unsigned u = __float_as_uint(x);
  const u32x2 a = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  x = vmax_raw(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const unsigned v = __float_as_uint(x);
  const u32x2 b = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return vmax_raw(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
// Two independent lanegroup_max chains interleaved (each one's swap fills the other's hazard wait).
__device__ __forceinline__ void lanegroup_max2(float& x, float& y) {
  const unsigned ux = __float_as_uint(x), uy = __float_as_uint(y);
  const u32x2 ax = __builtin_amdgcn_permlane16_swap(ux, ux, false, false);
  const u32x2 ay = __builtin_amdgcn_permlane16_swap(uy, uy, false, false);
  const float mx = vmax_raw(__uint_as_float(ax[0]), __uint_as_float(ax[1]));
  const float my = vmax_raw(__uint_as_float(ay[0]), __uint_as_float(ay[1]));
  const unsigned vx = __float_as_uint(mx), vy = __float_as_uint(my);
  const u32x2 bx = __builtin_amdgcn_permlane32_swap(vx, vx, false, false);
  const u32x2 by = __builtin_amdgcn_permlane32_swap(vy, vy, false, false);
  x = vmax_raw(__uint_as_float(bx[0]), __uint_as_float(bx[1]));
  y = vmax_raw(__uint_as_float(by[0]), __uint_as_float(by[1]));
}
__device__ __forceinline__ float lanegroup_sum(float x) {
  const unsigned u = __float_as_uint(x);
  const u32x2 a = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const unsigned v = __float_as_uint(x);
  const u32x2 b = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// DPP lane moves (gfx9 dpp_ctrl encodings), cheaper than a ds_bpermute shuffle: quad_perm [1,0,3,2]
// and [2,3,0,1] read lane ^ 1 and lane ^ 2; within a row of 16 lanes, row_ror:8 reads lane ^ 8 and
// row_ror:12 (a rotation by 12 to higher lanes) reads lane + 4 mod 16, which is lane ^ 4 for the
// lanes whose bit 2 is clear.
constexpr int kDppXor1 = 0xB1, kDppXor2 = 0x4E, kDppNext4 = 0x12C, kDppRor8 = 0x128;
template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), CTRL, 0xF, 0xF, false));
}
// Sum / max over the 64 lanes in the order of the xor butterfly 32, 16, 8, 4, 2, 1. The max reaches
// every lane; the sum is the butterfly's in lanes 0-3 (the others hold other partial sums).
__device__ __forceinline__ float wave_sum_lane0(float x) {
  unsigned u = __float_as_uint(x);
  u32x2 a = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  u = __float_as_uint(x);
  a = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  x += dpp<kDppRor8>(x);
  x += dpp<kDppNext4>(x);
  x += dpp<kDppXor2>(x);
  return x + dpp<kDppXor1>(x);
}
__device__ __forceinline__ float wave_max(float x) {
  unsigned u = __float_as_uint(x);
  u32x2 a = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  u = __float_as_uint(x);
  a = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  x = fmaxf(x, dpp<kDppRor8>(x));
  x = fmaxf(x, dpp<kDppNext4>(x));
  x = fmaxf(x, dpp<kDppXor2>(x));
  return fmaxf(x, dpp<kDppXor1>(x));
}

// ------------------------------------------------------------------------------------------------
// Element traits: fragments and the K32 matrix step
// ------------------------------------------------------------------------------------------------
template <typename T>
struct Elem;

template <>
struct Elem<bf16_t> {
  struct Frag {
    bf16x8 v;
  };
  static constexpr int kBytes = 2;
  __device__ static __forceinline__ float to_f(bf16_t x) { return bf2f(x); }
  __device__ static __forceinline__ bf16_t from_f(float x) { return f2bf(x); }
  __device__ static __forceinline__ f32x4 mma(const Frag& a, const Frag& b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a.v, b.v, c, 0, 0, 0);
  }
  __device__ static __forceinline__ Frag zero() {
    Frag f;
    f.v = bf16x8{};
    return f;
  }
  // 8 contiguous elements (16 bytes) -> fragment
  __device__ static __forceinline__ Frag load8(const bf16_t* p) {
    Frag f;
    f.v = *reinterpret_cast<const bf16x8*>(p);
    return f;
  }
  // two runs of 4 contiguous elements -> slots 0..3 and 4..7
  __device__ static __forceinline__ Frag load4x2(const bf16_t* p0, const bf16_t* p1) {
    bf16x4 a = *reinterpret_cast<const bf16x4*>(p0);
    bf16x4 b = *reinterpret_cast<const bf16x4*>(p1);
    Frag f;
    f.v = bf16x8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
    return f;
  }
  __device__ static __forceinline__ Frag from_f32(const float* s) {
    Frag f;
#pragma unroll
    for (int j = 0; j < 8; ++j) f.v[j] = (__bf16)s[j];
    return f;
  }
};

template <>
struct Elem<float> {
  struct Frag {
    float v[8];
  };
  static constexpr int kBytes = 4;
  __device__ static __forceinline__ float to_f(float x) { return x; }
  __device__ static __forceinline__ float from_f(float x) { return x; }
  __device__ static __forceinline__ f32x4 mma(const Frag& a, const Frag& b, f32x4 c) {
#pragma unroll
    for (int j = 0; j < 8; ++j) c = __builtin_amdgcn_mfma_f32_16x16x4f32(a.v[j], b.v[j], c, 0, 0, 0);
    return c;
  }
  __device__ static __forceinline__ Frag zero() {
    Frag f;
#pragma unroll
    for (int j = 0; j < 8; ++j) f.v[j] = 0.f;
    return f;
  }
  __device__ static __forceinline__ Frag load8(const float* p) {
    Frag f;
    const float4 a = reinterpret_cast<const float4*>(p)[0];
    const float4 b = reinterpret_cast<const float4*>(p)[1];
    f.v[0] = a.x; f.v[1] = a.y; f.v[2] = a.z; f.v[3] = a.w;
    f.v[4] = b.x; f.v[5] = b.y; f.v[6] = b.z; f.v[7] = b.w;
    return f;
  }
  __device__ static __forceinline__ Frag load4x2(const float* p0, const float* p1) {
    Frag f;
    const float4 a = *reinterpret_cast<const float4*>(p0);
    const float4 b = *reinterpret_cast<const float4*>(p1);
    f.v[0] = a.x; f.v[1] = a.y; f.v[2] = a.z; f.v[3] = a.w;
    f.v[4] = b.x; f.v[5] = b.y; f.v[6] = b.z; f.v[7] = b.w;
    return f;
  }
  __device__ static __forceinline__ Frag from_f32(const float* s) {
    Frag f;
#pragma unroll
    for (int j = 0; j < 8; ++j) f.v[j] = s[j];
    return f;
  }
};

// A 16-byte chunk of 16 / kBytes elements, the unit of global <-> LDS staging.
struct alignas(16) Chunk {
  uint32_t w[4];
};

__device__ __forceinline__ Chunk load_chunk(const void* p) { return *reinterpret_cast<const Chunk*>(p); }
__device__ __forceinline__ void store_chunk(void* p, const Chunk& c) { *reinterpret_cast<Chunk*>(p) = c; }
__device__ __forceinline__ Chunk zero_chunk() {
  Chunk c;
  c.w[0] = c.w[1] = c.w[2] = c.w[3] = 0u;
  return c;
}

// The rotation x c + y s (RoPE: x cos + rotate_half(x) sin; Givens: c a - s b, s a + c b) with the
// rounding points of eager tensor ops in the element type: each product is rounded to T, then the
// sum. For bf16 that is where the reference's per-op arithmetic rounds (the products of two bf16
// values are exact in fp32); contraction into an FMA is off, so fp32 elements get a separately
// rounded multiply and add as well.
template <typename T>
__device__ __forceinline__ float round_elem(float x) {
  return Elem<T>::to_f(Elem<T>::from_f(x));
}
template <typename T>
__device__ __forceinline__ float rot_round(float x, float c, float y, float s) {
#pragma clang fp contract(off)
  const float a = round_elem<T>(x * c);
  const float b = round_elem<T>(y * s);
  return round_elem<T>(a + b);
}

}  // namespace mote
