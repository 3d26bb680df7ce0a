// RoPE on P1/P2 and the Givens head-pair rotation of I~, fused with the split of the projection
// output [B, T, 3*H*D] (p1 | p2 | info per row) into the three [B, H, T, D] head views.
//
// Forward (mote/model/relation.py:37-68, 160-174):
//   RoPE, rotate-half convention: for k < D/2 with angle = float(pos) * inv_freq[k],
//     out_k = x_k c - x_{k+D/2} s,   out_{k+D/2} = x_{k+D/2} c + x_k s
//   Givens on the head pair (a, b) of pair index p with angle theta_p:
//     out_a = c a - s b,   out_b = s a + c b
//   c and s are rounded to the element type first (the reference casts its tables, :42, :165-166).
// Backward: the transposed rotations, plus d theta_p = sum over rows and d of
//   dout_a (-sin a - cos b) + dout_b (cos a - sin b)  (exact fp32 sin/cos, as autograd through the
//   cast gives), reduced deterministically: one partial per row and pair, then a fixed-order sum.
#include "common.hpp"
#include "params.hpp"

namespace mote {

struct RopeParams {
  const void* qkv;
  int64_t qkv_sb, qkv_sr;
  void* o1; int64_t o1_sb, o1_sh, o1_sr;
  void* o2; int64_t o2_sb, o2_sh, o2_sr;
  void* o3; int64_t o3_sb, o3_sh, o3_sr;
  const float* inv_freq;
  const float* theta;
  const float* inv_safe;    // never null: the tables, or any valid fp32 address when absent
  const float* theta_safe;
  int rope, givens;
  int B, T, H, D, pos0, parity;
};

template <typename T>
__device__ __forceinline__ float rnd(float x) {
  return Elem<T>::to_f(Elem<T>::from_f(x));
}

// Partner head and pair index of head `hd` for the Givens rotation; `first` is true for the
// first member (a) of the pair.
__device__ __forceinline__ void givens_pair(int hd, int H, int parity, int& pair, int& other, bool& first) {
  if (parity == 0) {
    pair = hd >> 1;
    first = (hd & 1) == 0;
    other = first ? hd + 1 : hd - 1;
  } else {
    // pairs (1,2), (3,4), ..., (H-1, 0)
    if (hd & 1) {
      first = true;
      pair = hd >> 1;
      other = (hd + 1) % H;
    } else {
      first = false;
      const int a = (hd + H - 1) % H;  // odd partner
      pair = a >> 1;
      other = a;
    }
  }
}

template <typename T>
__global__ void __launch_bounds__(256) rope_givens_fwd_kernel(const RopeParams p) {
  using E = Elem<T>;
  const int row = blockIdx.x;  // b * T + t
  const int b = row / p.T, t = row % p.T;
  const int HD = p.H * p.D, half = p.D / 2;
  const T* x = reinterpret_cast<const T*>(p.qkv) + int64_t(b) * p.qkv_sb + int64_t(t) * p.qkv_sr;
  const float pos = (float)(p.pos0 + t);
  // RoPE units: which in {0: p1, 1: p2} x head x k < D/2
  for (int u = threadIdx.x; u < HD; u += blockDim.x) {
    const int which = u / (p.H * half);
    const int rem = u % (p.H * half);
    const int hd = rem / half, k = rem % half;
    const T* xs = x + which * HD + hd * p.D;
    const float x0 = E::to_f(xs[k]), x1 = E::to_f(xs[k + half]);
    float o0 = x0, o1 = x1;
    if (p.inv_freq) {
      float s, c;
      sincosf(pos * p.inv_freq[k], &s, &c);
      c = rnd<T>(c);
      s = rnd<T>(s);
      o0 = x0 * c - x1 * s;
      o1 = x1 * c + x0 * s;
    }
    T* dst;
    if (which == 0) dst = reinterpret_cast<T*>(p.o1) + int64_t(b) * p.o1_sb + int64_t(hd) * p.o1_sh + int64_t(t) * p.o1_sr;
    else dst = reinterpret_cast<T*>(p.o2) + int64_t(b) * p.o2_sb + int64_t(hd) * p.o2_sh + int64_t(t) * p.o2_sr;
    dst[k] = E::from_f(o0);
    dst[k + half] = E::from_f(o1);
  }
  // Givens units: head x d
  for (int u = threadIdx.x; u < HD; u += blockDim.x) {
    const int hd = u / p.D, d = u % p.D;
    const T* xi = x + 2 * HD;
    const float self = E::to_f(xi[hd * p.D + d]);
    float out = self;
    if (p.theta) {
      int pair, other;
      bool first;
      givens_pair(hd, p.H, p.parity, pair, other, first);
      float s, c;
      sincosf(p.theta[pair], &s, &c);
      c = rnd<T>(c);
      s = rnd<T>(s);
      const float oth = E::to_f(xi[other * p.D + d]);
      out = first ? (c * self - s * oth) : (s * oth + c * self);
    }
    T* dst = reinterpret_cast<T*>(p.o3) + int64_t(b) * p.o3_sb + int64_t(hd) * p.o3_sh + int64_t(t) * p.o3_sr;
    dst[d] = E::from_f(out);
  }
}

struct RopeBwdParams {
  const void* qkv;
  int64_t qkv_sb, qkv_sr;
  int ioff;        // element offset of the I~ columns in a qkv row (2 H D, or 0 for I~ alone)
  const void* g1; int64_t g1_sb, g1_sh, g1_sr;
  const void* g2; int64_t g2_sb, g2_sh, g2_sr;
  const void* g3; int64_t g3_sb, g3_sh, g3_sr;
  void* dqkv;
  int64_t dq_sb, dq_sr;
  const float* inv_freq;
  const float* theta;
  const float* inv_safe;    // never null: the tables, or any valid fp32 address when absent
  const float* theta_safe;
  int rope, givens;
  float* partial;  // [blocks or rows][H/2]
  int B, T, H, D, pos0, parity;
};

template <typename T>
__global__ void __launch_bounds__(256) rope_givens_bwd_kernel(const RopeBwdParams p) {
  using E = Elem<T>;
  const int row = blockIdx.x;
  const int b = row / p.T, t = row % p.T;
  const int HD = p.H * p.D, half = p.D / 2;
  T* dx = reinterpret_cast<T*>(p.dqkv) + int64_t(b) * p.dq_sb + int64_t(t) * p.dq_sr;
  const float pos = (float)(p.pos0 + t);
  for (int u = threadIdx.x; u < HD; u += blockDim.x) {
    const int which = u / (p.H * half);
    const int rem = u % (p.H * half);
    const int hd = rem / half, k = rem % half;
    const T* gs;
    if (which == 0) gs = reinterpret_cast<const T*>(p.g1) + int64_t(b) * p.g1_sb + int64_t(hd) * p.g1_sh + int64_t(t) * p.g1_sr;
    else gs = reinterpret_cast<const T*>(p.g2) + int64_t(b) * p.g2_sb + int64_t(hd) * p.g2_sh + int64_t(t) * p.g2_sr;
    const float d0 = E::to_f(gs[k]), d1 = E::to_f(gs[k + half]);
    float r0 = d0, r1 = d1;
    if (p.inv_freq) {
      float s, c;
      sincosf(pos * p.inv_freq[k], &s, &c);
      c = rnd<T>(c);
      s = rnd<T>(s);
      r0 = d0 * c + d1 * s;
      r1 = d1 * c - d0 * s;
    }
    T* o = dx + which * HD + hd * p.D;
    o[k] = E::from_f(r0);
    o[k + half] = E::from_f(r1);
  }
  const T* xi = reinterpret_cast<const T*>(p.qkv) + int64_t(b) * p.qkv_sb + int64_t(t) * p.qkv_sr + p.ioff;
  const T* g3 = reinterpret_cast<const T*>(p.g3) + int64_t(b) * p.g3_sb + int64_t(t) * p.g3_sr;
  for (int u = threadIdx.x; u < HD; u += blockDim.x) {
    const int hd = u / p.D, d = u % p.D;
    const float gself = E::to_f(g3[int64_t(hd) * p.g3_sh + d]);
    float r = gself;
    if (p.theta) {
      int pair, other;
      bool first;
      givens_pair(hd, p.H, p.parity, pair, other, first);
      float s, c;
      sincosf(p.theta[pair], &s, &c);
      const float cr = rnd<T>(c), sr = rnd<T>(s);
      const float goth = E::to_f(g3[int64_t(other) * p.g3_sh + d]);
      // out_a = c a - s b, out_b = s a + c b  =>  da = c ga + s gb, db = -s ga + c gb
      r = first ? (cr * gself + sr * goth) : (cr * gself - sr * goth);
    }
    dx[2 * HD + hd * p.D + d] = E::from_f(r);
  }
  if (!p.theta) return;
  // d theta partials: one wave per pair, fixed-order reduction over d
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  const int npair = p.H / 2;
  for (int pr = wave; pr < npair; pr += nw) {
    int ha, hb;
    if (p.parity == 0) {
      ha = 2 * pr;
      hb = 2 * pr + 1;
    } else {
      ha = 2 * pr + 1;
      hb = (2 * pr + 2) % p.H;
    }
    float s, c;
    sincosf(p.theta[pr], &s, &c);
    float acc = 0.f;
    for (int d = lane; d < p.D; d += 64) {
      const float a = E::to_f(xi[ha * p.D + d]), bb = E::to_f(xi[hb * p.D + d]);
      const float ga = E::to_f(g3[int64_t(ha) * p.g3_sh + d]), gb = E::to_f(g3[int64_t(hb) * p.g3_sh + d]);
      acc += ga * (-s * a - c * bb) + gb * (c * a - s * bb);
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) acc += __shfl_xor(acc, off, 64);
    if (lane == 0) p.partial[int64_t(row) * npair + pr] = acc;
  }
}

// d theta: one block per pair; thread j sums partials j, j + 256, ... (eight loads in flight per
// batch), then each wave's lanes in a fixed butterfly (row swaps and DPP moves) and the four waves in
// order: the order is fixed, so the result is reproducible.
__global__ void __launch_bounds__(256) sum_partials_kernel(const float* partial, int rows, int npair, float* out) {
  __shared__ float red[4];
  const int tid = threadIdx.x, pr = blockIdx.x;
  float acc = 0.f;
  for (int base = 0; base < rows; base += 256 * 8) {
    float v[8];
#pragma unroll
    for (int m = 0; m < 8; ++m) v[m] = partial[int64_t(min(base + m * 256 + tid, rows - 1)) * npair + pr];
#pragma unroll
    for (int m = 0; m < 8; ++m)
      if (base + m * 256 + tid < rows) acc += v[m];
  }
  acc = wave_sum_lane0(acc);
  if ((tid & 63) == 0) red[tid >> 6] = acc;
  __syncthreads();
  if (tid == 0) out[pr] = (red[0] + red[1]) + (red[2] + red[3]);
}

// ------------------------------------------------------------------------------------------------
// Streaming kernels (16-byte chunks), used when D/2 is a multiple of the chunk and every view is
// 16-byte aligned. One thread per rotation unit of a row: a RoPE unit is a chunk of a head's first
// half with the same chunk of its second half (in p1 or p2), a Givens unit the same chunk of the two
// heads of a pair (in I~); the thread loads both chunks and stores both results, so every input
// chunk is loaded once and the two rows of a rotation meet in one thread. A row has
// U = 3 H cph / 2 units (cph chunks per head). A block has NS row slots of U threads and takes
// kRopeNR rows per slot (rows row0 + NS r + slot), so each thread keeps 2 kRopeNR chunk loads in
// flight; all of them are issued before any math (the table values first: loads complete in order),
// the RoPE factors of the block's rows and the Givens factors go through LDS, and the only barrier
// waits for them. Every unit reads its factors the same way (16-byte LDS reads, a per-lane base and
// row stride), so waves that hold both RoPE and Givens units run one instruction stream.
// ------------------------------------------------------------------------------------------------
constexpr int kRopeNR = 4;
constexpr int kRopeMaxThreads = 1024;

// The RoPE factors of a block's nr rows, [nr][D/2] cos then sin in LDS, rounded to the element type
// as the reference casts its tables. Entry i = r D/2 + k goes to thread i mod blockDim: a sincos of
// a large angle (positions in the thousands) takes the long argument reduction, so the entries are
// spread over the whole block rather than left to D/2 threads. The inverse frequencies of a thread's
// first two entries (`inv2`) are loaded before the chunk loads, so the sincos runs while they arrive.
// n / d for 0 <= n < 2^21 and d >= 1, given rd = rcp(d) (within 1 ulp): (n + 1/2) / d lies at least
// 1 / (2 d) from every integer, farther than the relative error (under 2^-22) moves it, so the
// truncation is floor(n / d). A few instructions where an integer division by a runtime value takes
// about twenty.
__device__ __forceinline__ int small_div(int n, float rd) { return int((float(n) + 0.5f) * rd); }

struct RopeInv {
  float v[2];
};
__device__ __forceinline__ RopeInv rope_inv(const float* inv_safe, int rope, int half) {
  const float rh = frcp(float(half));
  const int i0 = threadIdx.x, i1 = threadIdx.x + blockDim.x;
  RopeInv R;
  R.v[0] = inv_safe[(i0 - small_div(i0, rh) * half) * rope];
  R.v[1] = inv_safe[(i1 - small_div(i1, rh) * half) * rope];
  return R;
}
// Factors of positions pos0 + t0 + r, r < nr (rows past nrow repeat the last one).
template <typename T>
__device__ __forceinline__ void rope_factors(const RopeInv& inv2, const float* inv_safe, int rope, int pos0, int t0,
                                             int nr, int nrow, int half, float* tc, float* ts) {
  const float rh = frcp(float(half));
  const int n = nr * half;
  auto entry = [&](int i, float invk) {
    const int r = small_div(i, rh);
    const int t = t0 + min(r, nrow - 1);
    float sn, cs;
    sincosf((float)(pos0 + t) * invk, &sn, &cs);
    tc[i] = rope ? rnd<T>(cs) : 1.f;
    ts[i] = rope ? rnd<T>(sn) : 0.f;
  };
  // the first two entries take the preloaded frequencies; a value merged from a later load would make
  // the compiler wait for that load, the youngest, and so for every chunk load before it
  const int i0 = threadIdx.x, i1 = threadIdx.x + blockDim.x;
  if (i0 < n) entry(i0, inv2.v[0]);
  if (i1 < n) entry(i1, inv2.v[1]);
  for (int i = i1 + blockDim.x; i < n; i += blockDim.x) entry(i, inv_safe[(i - small_div(i, rh) * half) * rope]);
}

// A thread's rotation unit: tensor (0: p1, 1: p2, 2: I~), the two heads (one head for RoPE), the
// chunk k (RoPE: k < cph / 2, its partner k + cph / 2; Givens: the same chunk k < cph of both
// heads), the Givens pair, and the two chunks' positions in the [p1 | p2 | I~] row. Givens pairs
// (relation.py:150-174): even layers (0,1),(2,3)..., odd layers (1,2),...,(H-1,0); the first head of a
// pair gets c a - s b, the second s a + c b.
struct RopeUnit {
  int which, ha, hb, k, pair, ca, cb;
};
// Without branches: a wave can hold units of both kinds.
__device__ __forceinline__ RopeUnit rope_unit(int u, int H, int cph, int parity) {
  RopeUnit R;
  const int hch = cph / 2, ur = 2 * H * hch, cpt = H * cph;
  const bool rope_part = u < ur;
  // RoPE: u = (which H + head) hch + k; Givens: u - ur = pair cph + k
  const int v = rope_part ? u : u - ur;
  const int dv = rope_part ? hch : cph;
  const int hu = small_div(v, frcp(float(dv)));
  R.k = v - hu * dv;
  const int which = hu >= H ? 1 : 0;
  const int head = hu - which * H;
  R.which = rope_part ? which : 2;
  R.pair = rope_part ? 0 : hu;
  const int ga = parity == 0 ? 2 * hu : 2 * hu + 1;
  const int gb = parity == 0 ? 2 * hu + 1 : (2 * hu + 2 == H ? 0 : 2 * hu + 2);
  R.ha = rope_part ? head : ga;
  R.hb = rope_part ? head : gb;
  R.ca = rope_part ? which * cpt + head * cph + R.k : 2 * cpt + ga * cph + R.k;
  R.cb = rope_part ? R.ca + hch : 2 * cpt + gb * cph + R.k;
  return R;
}

// The Givens factors of the block's layer, EPC copies per pair, so that a Givens unit reads its chunk's
// factors the way a RoPE unit does (a factor row of stride 0): rounded cos, rounded sin, and for the
// backward the exact values [npair] cos, [npair] sin (d theta). `th` is the thread's theta, loaded
// before the chunk loads; the launcher keeps npair * EPC within the block.
template <typename T, int EPC>
__device__ __forceinline__ void givens_factors(float th, int givens, int npair, float* gc, float* gs, float* ge) {
  const int i = threadIdx.x;
  if (i < npair * EPC) {
    float sn, cs;
    sincosf(th, &sn, &cs);
    gc[i] = givens ? rnd<T>(cs) : 1.f;
    gs[i] = givens ? rnd<T>(sn) : 0.f;
    if (ge && i % EPC == 0) {
      ge[i / EPC] = givens ? cs : 1.f;
      ge[npair + i / EPC] = givens ? sn : 0.f;
    }
  }
}

// A unit's rotation factors: RoPE units read row rr of the block's table at their chunk, Givens units
// their pair's copies (row stride 0). Offsets in floats from the table's start; sin at + soff.
struct UnitFactors {
  int c0, stride, soff;
};
__device__ __forceinline__ UnitFactors unit_factors(const RopeUnit& R, int rpb, int half, int npair, int epc) {
  UnitFactors F;
  const bool rope_part = R.which < 2;
  const int gbase = 2 * rpb * half;  // the Givens copies follow the RoPE table
  F.c0 = rope_part ? R.k * epc : gbase + min(R.pair, npair - 1) * epc;
  F.stride = rope_part ? half : 0;
  F.soff = rope_part ? rpb * half : npair * epc;
  return F;
}

template <int EPC>
__device__ __forceinline__ void read_factors(const float* tab, const UnitFactors& F, int rr, float (&C)[EPC], float (&S)[EPC]) {
  const float* c = tab + F.c0 + rr * F.stride;
#pragma unroll
  for (int q = 0; q < EPC / 4; ++q) {
    const float4 cv = *reinterpret_cast<const float4*>(c + 4 * q);
    const float4 sv = *reinterpret_cast<const float4*>(c + F.soff + 4 * q);
    C[4 * q] = cv.x; C[4 * q + 1] = cv.y; C[4 * q + 2] = cv.z; C[4 * q + 3] = cv.w;
    S[4 * q] = sv.x; S[4 * q + 1] = sv.y; S[4 * q + 2] = sv.z; S[4 * q + 3] = sv.w;
  }
}

typedef __attribute__((ext_vector_type(2))) float f32x2;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2;

// Two fp32 values as two bf16 in one word (lo = a), one v_cvt_pk_bf16_f32 for both.
__device__ __forceinline__ uint32_t pack_bf16(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, bf16x2));
}
__device__ __forceinline__ float bf_lo(uint32_t u) { return __uint_as_float(u << 16); }
__device__ __forceinline__ float bf_hi(uint32_t u) { return __uint_as_float(u & 0xffff0000u); }

// Forward rotation of a chunk pair with the element type's rounding points (rot_round):
// out_a = x_a C - x_b S, out_b = x_b C + x_a S, every product and the sum rounded to T. For bf16 the
// roundings of element pairs share one conversion.
template <typename T, int EPC>
__device__ __forceinline__ void rot_chunks(const Chunk& xa, const Chunk& xb, const float (&C)[EPC], const float (&S)[EPC],
                                           Chunk& oa, Chunk& ob) {
#pragma clang fp contract(off)
  if constexpr (sizeof(T) == 2) {
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float a0 = bf_lo(xa.w[w]), a1 = bf_hi(xa.w[w]), b0 = bf_lo(xb.w[w]), b1 = bf_hi(xb.w[w]);
      const float c0 = C[2 * w], c1 = C[2 * w + 1], s0 = S[2 * w], s1 = S[2 * w + 1];
      const uint32_t ac = pack_bf16(a0 * c0, a1 * c1), bs = pack_bf16(b0 * -s0, b1 * -s1);
      const uint32_t bc = pack_bf16(b0 * c0, b1 * c1), as = pack_bf16(a0 * s0, a1 * s1);
      oa.w[w] = pack_bf16(bf_lo(ac) + bf_lo(bs), bf_hi(ac) + bf_hi(bs));
      ob.w[w] = pack_bf16(bf_lo(bc) + bf_lo(as), bf_hi(bc) + bf_hi(as));
    }
  } else {
    const float* ea = reinterpret_cast<const float*>(&xa);
    const float* eb = reinterpret_cast<const float*>(&xb);
    float* ya = reinterpret_cast<float*>(&oa);
    float* yb = reinterpret_cast<float*>(&ob);
#pragma unroll
    for (int e = 0; e < EPC; ++e) {
      ya[e] = rot_round<T>(ea[e], C[e], eb[e], -S[e]);
      yb[e] = rot_round<T>(eb[e], C[e], ea[e], S[e]);
    }
  }
}

// Backward rotation (the transpose, fp32 arithmetic, one rounding at the end):
// d_a = g_a C + g_b S, d_b = g_b C - g_a S.
template <typename T, int EPC>
__device__ __forceinline__ void rot_chunks_t(const Chunk& ga, const Chunk& gb, const float (&C)[EPC], const float (&S)[EPC],
                                             Chunk& oa, Chunk& ob) {
  if constexpr (sizeof(T) == 2) {
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float a0 = bf_lo(ga.w[w]), a1 = bf_hi(ga.w[w]), b0 = bf_lo(gb.w[w]), b1 = bf_hi(gb.w[w]);
      const float c0 = C[2 * w], c1 = C[2 * w + 1], s0 = S[2 * w], s1 = S[2 * w + 1];
      oa.w[w] = pack_bf16(a0 * c0 + b0 * s0, a1 * c1 + b1 * s1);
      ob.w[w] = pack_bf16(b0 * c0 + a0 * -s0, b1 * c1 + a1 * -s1);
    }
  } else {
    const float* ea = reinterpret_cast<const float*>(&ga);
    const float* eb = reinterpret_cast<const float*>(&gb);
    float* ya = reinterpret_cast<float*>(&oa);
    float* yb = reinterpret_cast<float*>(&ob);
#pragma unroll
    for (int e = 0; e < EPC; ++e) {
      ya[e] = ea[e] * C[e] + eb[e] * S[e];
      yb[e] = eb[e] * C[e] + ea[e] * -S[e];
    }
  }
}

template <typename T>
__global__ void __launch_bounds__(kRopeMaxThreads) rope_givens_fwd_stream_kernel(const RopeParams p, int NS) {
  constexpr int EPC = 16 / sizeof(T);
  // RoPE factors [rpb][D/2] cos, then sin; the Givens copies [npair][EPC] cos, then sin
  extern __shared__ float rope_tab[];
  const int tid = threadIdx.x;
  const int H = p.H, D = p.D, half = D / 2, npair = H / 2, cph = D / EPC, hch = cph / 2;
  const int U = 3 * H * cph / 2, rpb = NS * kRopeNR;
  const int b = blockIdx.y, t0 = blockIdx.x * rpb;  // positions t0 .. t0 + nrow - 1 of sequence b
  const int nrow = min(rpb, p.T - t0);
  const bool act = tid < NS * U;
  const int slot = act ? small_div(tid, frcp(float(U))) : 0;
  const RopeUnit R = rope_unit(act ? tid - slot * U : 0, H, cph, p.parity);

  // table values first (indices by multiplication with the 0/1 flags: a select becomes a branch)
  const RopeInv inv2 = rope_inv(p.inv_safe, p.rope, half);
  const float th = p.theta_safe[min(tid / EPC, npair - 1) * p.givens];
  // Keeps these table loads ahead of the chunk loads: left alone, the compiler sinks them to their
  // use (the factor loop, after every chunk load) and, loads completing in order, the sincos then
  // waits for all the chunks.
  asm volatile("" ::: "memory");
  // the unit's rows (clamped to the block's last row)
  int rt[kRopeNR];
  Chunk xa[kRopeNR], xb[kRopeNR];
  const T* q = reinterpret_cast<const T*>(p.qkv) + int64_t(b) * p.qkv_sb;
#pragma unroll
  for (int r = 0; r < kRopeNR; ++r) {
    rt[r] = t0 + min(NS * r + slot, nrow - 1);
    const T* base = q + int64_t(rt[r]) * p.qkv_sr;
    xa[r] = load_chunk(base + R.ca * EPC);
    xb[r] = load_chunk(base + R.cb * EPC);
  }
  float* tc = rope_tab;
  float* ts = tc + rpb * half;
  rope_factors<T>(inv2, p.inv_safe, p.rope, p.pos0, t0, rpb, nrow, half, tc, ts);
  givens_factors<T, EPC>(th, p.givens, npair, ts + rpb * half, ts + rpb * half + npair * EPC, nullptr);
  __syncthreads();
  if (!act) return;

  // RoPE: out_k = x_k c - x_{k+D/2} s, out_{k+D/2} = x_{k+D/2} c + x_k s; Givens: out_a = c a - s b,
  // out_b = s a + c b
  const bool rope_part = R.which < 2;
  T* obase;
  int64_t osb, osh, osr;
  if (R.which == 0) {
    obase = reinterpret_cast<T*>(p.o1); osb = p.o1_sb; osh = p.o1_sh; osr = p.o1_sr;
  } else if (R.which == 1) {
    obase = reinterpret_cast<T*>(p.o2); osb = p.o2_sb; osh = p.o2_sh; osr = p.o2_sr;
  } else {
    obase = reinterpret_cast<T*>(p.o3); osb = p.o3_sb; osh = p.o3_sh; osr = p.o3_sr;
  }
  T* oa = obase + int64_t(b) * osb + int64_t(R.ha) * osh + R.k * EPC;
  T* ob = rope_part ? oa + hch * EPC : obase + int64_t(b) * osb + int64_t(R.hb) * osh + R.k * EPC;
  const UnitFactors F = unit_factors(R, rpb, half, npair, EPC);
#pragma unroll
  for (int r = 0; r < kRopeNR; ++r) {
    const int rr = NS * r + slot;
    if (rr >= nrow) break;
    float C[EPC], S[EPC];
    read_factors<EPC>(rope_tab, F, rr, C, S);
    Chunk outa, outb;
    rot_chunks<T, EPC>(xa[r], xb[r], C, S, outa, outb);
    const int64_t off = int64_t(rt[r]) * osr;
    store_chunk(oa + off, outa);
    store_chunk(ob + off, outb);
  }
}

// The backward's block: the RoPE units fill the first waves, the Givens units start at a wave boundary
// (rope_bwd_threads), so a wave holds units of one kind and only the Givens waves load the I~ inputs
// that d theta needs. One row slot of kRopeNR rows.
__host__ __device__ inline int rope_bwd_givens_lane0(int H, int cph) { return (H * cph + 63) / 64 * 64; }
static inline int rope_bwd_threads(int H, int cph) { return rope_bwd_givens_lane0(H, cph) + ((H / 2) * cph + 63) / 64 * 64; }

template <typename T>
__global__ void __launch_bounds__(kRopeMaxThreads) rope_givens_bwd_stream_kernel(const RopeBwdParams p) {
  using E = Elem<T>;
  constexpr int EPC = 16 / sizeof(T);
  // RoPE factors [rpb][D/2] cos, then sin; the Givens copies [npair][EPC] cos, then sin; the exact
  // Givens cos, sin [npair] each; then [threads] d theta
  extern __shared__ float rope_tab[];
  const int tid = threadIdx.x;
  const int H = p.H, D = p.D, half = D / 2, npair = H / 2, cph = D / EPC, hch = cph / 2;
  const int rpb = kRopeNR, ur = 2 * H * hch, ug = npair * cph;
  const int b = blockIdx.y, t0 = blockIdx.x * rpb;  // positions t0 .. t0 + nrow - 1 of sequence b
  const int nrow = min(rpb, p.T - t0);
  float* tc = rope_tab;
  float* ts = tc + rpb * half;
  float* gtab = ts + rpb * half;
  float* gexact = gtab + 2 * npair * EPC;
  float* red = gexact + 2 * npair;
  const int g0lane = rope_bwd_givens_lane0(H, cph);
  const bool gwave = __builtin_amdgcn_readfirstlane(tid >> 6) * 64 >= g0lane;  // wave-uniform
  const bool act = gwave ? tid - g0lane < ug : tid < ur;
  // idle lanes take a unit of their wave's kind, so their addresses stay valid
  const int u = gwave ? ur + min(tid - g0lane, ug - 1) : min(tid, ur - 1);
  const RopeUnit R = rope_unit(u, H, cph, p.parity);

  const RopeInv inv2 = rope_inv(p.inv_safe, p.rope, half);
  const float th = p.theta_safe[min(tid / EPC, npair - 1) * p.givens];
  // Keeps these table loads ahead of the chunk loads: left alone, the compiler sinks them to their
  // use (the factor loop, after every chunk load) and, loads completing in order, the sincos then
  // waits for all the chunks.
  asm volatile("" ::: "memory");
  // gradient chunks of the unit, from the view of its tensor
  const T* gb;
  int64_t gsb, gsh, gsr;
  if (R.which == 0) {
    gb = reinterpret_cast<const T*>(p.g1); gsb = p.g1_sb; gsh = p.g1_sh; gsr = p.g1_sr;
  } else if (R.which == 1) {
    gb = reinterpret_cast<const T*>(p.g2); gsb = p.g2_sb; gsh = p.g2_sh; gsr = p.g2_sr;
  } else {
    gb = reinterpret_cast<const T*>(p.g3); gsb = p.g3_sb; gsh = p.g3_sh; gsr = p.g3_sr;
  }
  const T* gpa = gb + int64_t(b) * gsb + int64_t(R.ha) * gsh + R.k * EPC;
  const T* gpb = R.which < 2 ? gpa + hch * EPC : gb + int64_t(b) * gsb + int64_t(R.hb) * gsh + R.k * EPC;
  int rt[kRopeNR];
#pragma unroll
  for (int r = 0; r < kRopeNR; ++r) rt[r] = t0 + min(r, nrow - 1);
  // the pair's I~ inputs (d theta), loaded by the Givens waves only, ahead of the gradients
  Chunk g0[kRopeNR], g1[kRopeNR], x0[kRopeNR], x1[kRopeNR];
  if (gwave && p.givens) {
    const T* xq = reinterpret_cast<const T*>(p.qkv) + int64_t(b) * p.qkv_sb + p.ioff + R.k * EPC;
#pragma unroll
    for (int r = 0; r < kRopeNR; ++r) {
      const T* xr = xq + int64_t(rt[r]) * p.qkv_sr;
      x0[r] = load_chunk(xr + R.ha * D);
      x1[r] = load_chunk(xr + R.hb * D);
    }
  }
#pragma unroll
  for (int r = 0; r < kRopeNR; ++r) {
    const int64_t go = int64_t(rt[r]) * gsr;
    g0[r] = load_chunk(gpa + go);
    g1[r] = load_chunk(gpb + go);
  }
  rope_factors<T>(inv2, p.inv_safe, p.rope, p.pos0, t0, rpb, nrow, half, tc, ts);
  givens_factors<T, EPC>(th, p.givens, npair, gtab, gtab + npair * EPC, gexact);
  __syncthreads();

  // RoPE^T: dx_k = d_k c + d_{k+D/2} s, dx_{k+D/2} = d_{k+D/2} c - d_k s; Givens^T: da = c ga + s gb,
  // db = c gb - s ga
  const bool rope_part = R.which < 2;
  const bool dth_unit = act && !rope_part && p.givens;
  const int pr = min(R.pair, npair - 1);
  const float ce = gexact[pr], se = gexact[npair + pr];  // exact: the derivative
  T* da_out = reinterpret_cast<T*>(p.dqkv) + int64_t(b) * p.dq_sb + R.ca * EPC;
  T* db_out = reinterpret_cast<T*>(p.dqkv) + int64_t(b) * p.dq_sb + R.cb * EPC;
  const UnitFactors F = unit_factors(R, rpb, half, npair, EPC);
  float acc = 0.f;
#pragma unroll
  for (int r = 0; r < kRopeNR; ++r) {
    if (r >= nrow) break;
    float C[EPC], S[EPC];
    read_factors<EPC>(rope_tab, F, r, C, S);
    Chunk outa, outb;
    rot_chunks_t<T, EPC>(g0[r], g1[r], C, S, outa, outb);
    if (act) {
      const int64_t off = int64_t(rt[r]) * p.dq_sr;
      store_chunk(da_out + off, outa);
      store_chunk(db_out + off, outb);
    }
    if (dth_unit) {
      // d theta of the pair: ga (-s a - c b) + gb (c a - s b), exact s, c
      const T* ea = reinterpret_cast<const T*>(&x0[r]);
      const T* eb = reinterpret_cast<const T*>(&x1[r]);
      const T* e0 = reinterpret_cast<const T*>(&g0[r]);
      const T* e1 = reinterpret_cast<const T*>(&g1[r]);
#pragma unroll
      for (int e = 0; e < EPC; ++e) {
        const float a = E::to_f(ea[e]), bb = E::to_f(eb[e]);
        const float da = E::to_f(e0[e]), db = E::to_f(e1[e]);
        acc += da * (-se * a - ce * bb) + db * (ce * a - se * bb);
      }
    }
  }
  if (!p.givens) return;
  // one partial per block and pair: the pair's units in a fixed order (chunk)
  red[tid] = dth_unit ? acc : 0.f;
  __syncthreads();
  for (int q = tid; q < npair; q += blockDim.x) {
    float s2 = 0.f;
    for (int k = 0; k < cph; ++k) s2 += red[g0lane + q * cph + k];
    p.partial[(int64_t(b) * gridDim.x + blockIdx.x) * npair + q] = s2;
  }
}

static bool al16(const void* ptr, int64_t s0, int64_t s1, int64_t s2, int es) {
  const int64_t m = 16 / es;
  return (reinterpret_cast<uintptr_t>(ptr) % 16 == 0) && s0 % m == 0 && s1 % m == 0 && s2 % m == 0;
}

static bool aligned16(const mote_rope_givens_args* a) {
  const int es = a->dtype == MOTE_BF16 ? 2 : 4;
  return al16(a->qkv, a->qkv_sb, a->qkv_sr, 0, es) && al16(a->p1.data, a->p1.stride_b, a->p1.stride_h, a->p1.stride_r, es) &&
         al16(a->p2.data, a->p2.stride_b, a->p2.stride_h, a->p2.stride_r, es) &&
         al16(a->info.data, a->info.stride_b, a->info.stride_h, a->info.stride_r, es);
}

static bool aligned16_bwd(const mote_rope_givens_bwd_args* a) {
  const int es = a->dtype == MOTE_BF16 ? 2 : 4;
  return al16(a->qkv, a->qkv_sb, a->qkv_sr, 0, es) && al16(a->dqkv, a->dqkv_sb, a->dqkv_sr, 0, es) &&
         al16(a->dp1.data, a->dp1.stride_b, a->dp1.stride_h, a->dp1.stride_r, es) &&
         al16(a->dp2.data, a->dp2.stride_b, a->dp2.stride_h, a->dp2.stride_r, es) &&
         al16(a->dinfo.data, a->dinfo.stride_b, a->dinfo.stride_h, a->dinfo.stride_r, es);
}

// Streaming kernels' shape: chunks of EPC elements that split each head in halves, units per row
// (3 H cph / 2) and row slots per block. One slot: measured at the Mote-96M shape (bf16, 144 units),
// two slots of four rows ran the forward 4 % and the backward 40 % slower than one (more RoPE
// factors per block, fewer blocks in flight).
static bool stream_shape(int H, int D, int epc, int& units, int& NS) {
  if (D % (2 * epc) != 0) return false;
  units = 3 * H * (D / epc) / 2;
  NS = 1;
  return units <= kRopeMaxThreads && units >= (H / 2) * epc;  // the block writes the Givens copies
}

static int check_rope_common(int dtype, int B, int T, int H, int D, const void* qkv) {
  if (dtype != MOTE_F32 && dtype != MOTE_BF16) return set_error(MOTE_ERR_ARGUMENT, "rope_givens: bad dtype %d", dtype);
  if (!qkv) return set_error(MOTE_ERR_ARGUMENT, "rope_givens: null qkv");
  if (B <= 0 || T < 0 || H <= 0 || H % 2 || D <= 0 || D % 2) return set_error(MOTE_ERR_SHAPE, "rope_givens: bad sizes B=%d T=%d H=%d D=%d", B, T, H, D);
  return MOTE_OK;
}

int launch_rope_givens_fwd(const mote_rope_givens_args* a, hipStream_t stream) {
  if (!a) return set_error(MOTE_ERR_ARGUMENT, "rope_givens: null args");
  int rc = check_rope_common(a->dtype, a->B, a->T, a->H, a->D, a->qkv);
  if (rc) return rc;
  if (!a->p1.data || !a->p2.data || !a->info.data) return set_error(MOTE_ERR_ARGUMENT, "rope_givens: null output");
  if (a->T == 0) return MOTE_OK;
  RopeParams p;
  p.qkv = a->qkv; p.qkv_sb = a->qkv_sb; p.qkv_sr = a->qkv_sr;
  p.o1 = a->p1.data; p.o1_sb = a->p1.stride_b; p.o1_sh = a->p1.stride_h; p.o1_sr = a->p1.stride_r;
  p.o2 = a->p2.data; p.o2_sb = a->p2.stride_b; p.o2_sh = a->p2.stride_h; p.o2_sr = a->p2.stride_r;
  p.o3 = a->info.data; p.o3_sb = a->info.stride_b; p.o3_sh = a->info.stride_h; p.o3_sr = a->info.stride_r;
  p.inv_freq = a->inv_freq; p.theta = a->theta;
  p.rope = a->inv_freq != nullptr;
  p.givens = a->theta != nullptr;
  p.inv_safe = p.rope ? a->inv_freq : reinterpret_cast<const float*>(a->qkv);
  p.theta_safe = p.givens ? a->theta : reinterpret_cast<const float*>(a->qkv);
  p.B = a->B; p.T = a->T; p.H = a->H; p.D = a->D; p.pos0 = a->pos0; p.parity = a->layer_parity & 1;
  const int rows = a->B * a->T;
  const int epc = a->dtype == MOTE_BF16 ? 8 : 4;
  int units, NS;
  const bool vec = stream_shape(a->H, a->D, epc, units, NS) && aligned16(a);
  if (vec) {
    const dim3 blocks((a->T + NS * kRopeNR - 1) / (NS * kRopeNR), a->B);  // row groups of each sequence
    const int threads = (NS * units + 63) / 64 * 64;
    const size_t lds = (size_t(2) * NS * kRopeNR * (a->D / 2) + size_t(2) * (a->H / 2) * epc) * sizeof(float);
    if (a->dtype == MOTE_BF16)
      hipLaunchKernelGGL(rope_givens_fwd_stream_kernel<bf16_t>, blocks, dim3(threads), lds, stream, p, NS);
    else
      hipLaunchKernelGGL(rope_givens_fwd_stream_kernel<float>, blocks, dim3(threads), lds, stream, p, NS);
  } else if (a->dtype == MOTE_BF16) {
    hipLaunchKernelGGL(rope_givens_fwd_kernel<bf16_t>, dim3(rows), dim3(256), 0, stream, p);
  } else {
    hipLaunchKernelGGL(rope_givens_fwd_kernel<float>, dim3(rows), dim3(256), 0, stream, p);
  }
  return check_launch("rope_givens_fwd");
}

size_t rope_givens_bwd_workspace_bytes(const mote_rope_givens_bwd_args* a) {
  return size_t(a->B) * size_t(a->T) * size_t(a->H / 2) * sizeof(float) + 256;
}

int launch_rope_givens_bwd(const mote_rope_givens_bwd_args* a, hipStream_t stream) {
  if (!a) return set_error(MOTE_ERR_ARGUMENT, "rope_givens_bwd: null args");
  int rc = check_rope_common(a->dtype, a->B, a->T, a->H, a->D, a->qkv);
  if (rc) return rc;
  if (!a->dp1.data || !a->dp2.data || !a->dinfo.data || !a->dqkv) return set_error(MOTE_ERR_ARGUMENT, "rope_givens_bwd: null tensor");
  if (a->theta && !a->dtheta) return set_error(MOTE_ERR_ARGUMENT, "rope_givens_bwd: theta given without dtheta");
  if (a->theta && (a->workspace == nullptr || a->workspace_bytes < rope_givens_bwd_workspace_bytes(a)))
    return set_error(MOTE_ERR_WORKSPACE, "rope_givens_bwd: workspace too small");
  if (a->T == 0) return MOTE_OK;
  RopeBwdParams p;
  p.qkv = a->qkv; p.qkv_sb = a->qkv_sb; p.qkv_sr = a->qkv_sr;
  p.ioff = a->qkv_info_only ? 0 : 2 * a->H * a->D;
  p.g1 = a->dp1.data; p.g1_sb = a->dp1.stride_b; p.g1_sh = a->dp1.stride_h; p.g1_sr = a->dp1.stride_r;
  p.g2 = a->dp2.data; p.g2_sb = a->dp2.stride_b; p.g2_sh = a->dp2.stride_h; p.g2_sr = a->dp2.stride_r;
  p.g3 = a->dinfo.data; p.g3_sb = a->dinfo.stride_b; p.g3_sh = a->dinfo.stride_h; p.g3_sr = a->dinfo.stride_r;
  p.dqkv = a->dqkv; p.dq_sb = a->dqkv_sb; p.dq_sr = a->dqkv_sr;
  p.inv_freq = a->inv_freq; p.theta = a->theta;
  p.rope = a->inv_freq != nullptr;
  p.givens = a->theta != nullptr;
  p.inv_safe = p.rope ? a->inv_freq : reinterpret_cast<const float*>(a->qkv);
  p.theta_safe = p.givens ? a->theta : reinterpret_cast<const float*>(a->qkv);
  p.partial = reinterpret_cast<float*>(a->workspace);
  p.B = a->B; p.T = a->T; p.H = a->H; p.D = a->D; p.pos0 = a->pos0; p.parity = a->layer_parity & 1;
  const int rows = a->B * a->T;
  const int epc = a->dtype == MOTE_BF16 ? 8 : 4;
  int units, NS;
  const int threads = rope_bwd_threads(a->H, a->D / epc);
  const bool vec = stream_shape(a->H, a->D, epc, units, NS) && threads <= kRopeMaxThreads && aligned16_bwd(a);
  const int groups = (a->T + kRopeNR - 1) / kRopeNR;  // row groups of each sequence
  const dim3 blocks = vec ? dim3(groups, a->B) : dim3(rows);
  if (vec) {
    const size_t lds = (size_t(2) * kRopeNR * (a->D / 2) + size_t(2) * (a->H / 2) * (epc + 1) + size_t(threads)) *
                       sizeof(float);
    if (a->dtype == MOTE_BF16)
      hipLaunchKernelGGL(rope_givens_bwd_stream_kernel<bf16_t>, blocks, dim3(threads), lds, stream, p);
    else
      hipLaunchKernelGGL(rope_givens_bwd_stream_kernel<float>, blocks, dim3(threads), lds, stream, p);
  } else if (a->dtype == MOTE_BF16) {
    hipLaunchKernelGGL(rope_givens_bwd_kernel<bf16_t>, dim3(rows), dim3(256), 0, stream, p);
  } else {
    hipLaunchKernelGGL(rope_givens_bwd_kernel<float>, dim3(rows), dim3(256), 0, stream, p);
  }
  rc = check_launch("rope_givens_bwd");
  if (rc || !a->theta) return rc;
  const int nparts = int(blocks.x * blocks.y);  // one partial per block (the per-row kernel: one per row)
  hipLaunchKernelGGL(sum_partials_kernel, dim3(a->H / 2), dim3(256), 0, stream, p.partial, nparts, a->H / 2, a->dtheta);
  return check_launch("rope_givens_bwd/sum");
}

}  // namespace mote
