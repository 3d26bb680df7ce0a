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
  const void* g1; int64_t g1_sb, g1_sh, g1_sr;
  const void* g2; int64_t g2_sb, g2_sh, g2_sr;
  const void* g3; int64_t g3_sb, g3_sh, g3_sr;
  void* dqkv;
  int64_t dq_sb, dq_sr;
  const float* inv_freq;
  const float* theta;
  float* partial;  // [B*T, H/2]
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
  const T* xi = reinterpret_cast<const T*>(p.qkv) + int64_t(b) * p.qkv_sb + int64_t(t) * p.qkv_sr + 2 * HD;
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

__global__ void __launch_bounds__(256) sum_partials_kernel(const float* partial, int rows, int npair, float* out) {
  // one wave per pair (pairs strided over the waves): fixed-order strided sums, then a fixed tree
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  for (int pr = blockIdx.x * 4 + wave; pr < npair; pr += gridDim.x * 4) {
    float acc = 0.f;
    for (int r = lane; r < rows; r += 64) acc += partial[int64_t(r) * npair + pr];
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) acc += __shfl_xor(acc, off, 64);
    if (lane == 0) out[pr] = acc;
  }
}

// ------------------------------------------------------------------------------------------------
// Vectorised kernels (16-byte chunks), used when D/2 is a multiple of the chunk. A block handles
// kRopeRows rows; each thread loops over (row, unit) pairs: a RoPE unit is one chunk k..k+EPC of
// the first half of one head, for p1 and p2 together (the angles are shared); a Givens unit is one
// chunk of both heads of one pair.
// ------------------------------------------------------------------------------------------------
constexpr int kRopeRows = 8;

template <typename T>
__device__ __forceinline__ void rope_chunk_fwd(const T* x, T* o, int half, int k0, const float* ang_c, const float* ang_s) {
  using E = Elem<T>;
  constexpr int EPC = 16 / sizeof(T);
  const Chunk a = load_chunk(x + k0), b = load_chunk(x + half + k0);
  const T* ea = reinterpret_cast<const T*>(&a);
  const T* eb = reinterpret_cast<const T*>(&b);
  Chunk ra, rb;
  T* oa = reinterpret_cast<T*>(&ra);
  T* ob = reinterpret_cast<T*>(&rb);
#pragma unroll
  for (int e = 0; e < EPC; ++e) {
    const float x0 = E::to_f(ea[e]), x1 = E::to_f(eb[e]);
    oa[e] = E::from_f(x0 * ang_c[e] - x1 * ang_s[e]);
    ob[e] = E::from_f(x1 * ang_c[e] + x0 * ang_s[e]);
  }
  store_chunk(o + k0, ra);
  store_chunk(o + half + k0, rb);
}

// The block's RoPE factors for its kRopeRows positions and the Givens factors of every head pair,
// once per block in LDS (the angles do not depend on the head): rounded to the element type as the
// reference casts its tables. Returns through `tc` / `ts` ([kRopeRows][half]) and `gc` / `gs`
// ([H/2]); the exact fp32 Givens sin/cos go to `gce` / `gse` when those are given.
template <typename T>
__device__ __forceinline__ void rope_tables_lds(const float* inv_freq, const float* theta, int pos0, int row0, int T_,
                                                int half, int npair, float* tc, float* ts, float* gc, float* gs,
                                                float* gce, float* gse) {
  for (int q = threadIdx.x; q < kRopeRows * half; q += blockDim.x) {
    const int rl = q / half, k = q % half;
    float c = 1.f, sn = 0.f;
    if (inv_freq) {
      const int t = (row0 + rl) % T_;
      sincosf((float)(pos0 + t) * inv_freq[k], &sn, &c);
      c = rnd<T>(c);
      sn = rnd<T>(sn);
    }
    tc[q] = c;
    ts[q] = sn;
  }
  for (int q = threadIdx.x; q < npair; q += blockDim.x) {
    float c = 1.f, sn = 0.f;
    if (theta) sincosf(theta[q], &sn, &c);
    if (gce) {
      gce[q] = c;
      gse[q] = sn;
    }
    gc[q] = rnd<T>(c);
    gs[q] = rnd<T>(sn);
  }
  __syncthreads();
}

constexpr int kRopeMaxHalf = 64;   // D <= 128
constexpr int kRopeMaxPairs = 64;  // H <= 128

template <typename T>
__global__ void __launch_bounds__(256) rope_givens_fwd_vec_kernel(const RopeParams p) {
  using E = Elem<T>;
  constexpr int EPC = 16 / sizeof(T);
  __shared__ __align__(16) float tc[kRopeRows * kRopeMaxHalf], ts[kRopeRows * kRopeMaxHalf];
  __shared__ float gc[kRopeMaxPairs], gs[kRopeMaxPairs];
  const int HD = p.H * p.D, half = p.D / 2;
  const int ur = p.H * (half / EPC);          // RoPE units per row
  const int ug = (p.H / 2) * (p.D / EPC);     // Givens units per row
  const int upr = ur + ug;
  const int rows = p.B * p.T;
  const int row0 = blockIdx.x * kRopeRows;
  rope_tables_lds<T>(p.inv_freq, p.theta, p.pos0, row0, p.T, half, p.H / 2, tc, ts, gc, gs, nullptr, nullptr);
  for (int u = threadIdx.x; u < kRopeRows * upr; u += blockDim.x) {
    const int rl = u / upr, k = u % upr;
    const int row = row0 + rl;
    if (row >= rows) break;
    const int b = row / p.T, t = row % p.T;
    const T* x = reinterpret_cast<const T*>(p.qkv) + int64_t(b) * p.qkv_sb + int64_t(t) * p.qkv_sr;
    if (k < ur) {
      const int hd = k / (half / EPC), k0 = (k % (half / EPC)) * EPC;
      const float* cs = tc + rl * half + k0;
      const float* sn = ts + rl * half + k0;
      T* o1 = reinterpret_cast<T*>(p.o1) + int64_t(b) * p.o1_sb + int64_t(hd) * p.o1_sh + int64_t(t) * p.o1_sr;
      T* o2 = reinterpret_cast<T*>(p.o2) + int64_t(b) * p.o2_sb + int64_t(hd) * p.o2_sh + int64_t(t) * p.o2_sr;
      rope_chunk_fwd<T>(x + hd * p.D, o1, half, k0, cs, sn);
      rope_chunk_fwd<T>(x + HD + hd * p.D, o2, half, k0, cs, sn);
    } else {
      const int kg = k - ur;
      const int pr = kg / (p.D / EPC), d0 = (kg % (p.D / EPC)) * EPC;
      int ha, hb;
      if (p.parity == 0) {
        ha = 2 * pr;
        hb = 2 * pr + 1;
      } else {
        ha = 2 * pr + 1;
        hb = (2 * pr + 2) % p.H;
      }
      const T* xi = x + 2 * HD;
      const Chunk ca = load_chunk(xi + ha * p.D + d0), cb = load_chunk(xi + hb * p.D + d0);
      Chunk ra = ca, rb = cb;
      if (p.theta) {
        const float c = gc[pr], sn = gs[pr];
        const T* ea = reinterpret_cast<const T*>(&ca);
        const T* eb = reinterpret_cast<const T*>(&cb);
        T* oa = reinterpret_cast<T*>(&ra);
        T* ob = reinterpret_cast<T*>(&rb);
#pragma unroll
        for (int e = 0; e < EPC; ++e) {
          const float a = E::to_f(ea[e]), bb = E::to_f(eb[e]);
          oa[e] = E::from_f(c * a - sn * bb);
          ob[e] = E::from_f(sn * a + c * bb);
        }
      }
      T* o3 = reinterpret_cast<T*>(p.o3) + int64_t(b) * p.o3_sb + int64_t(t) * p.o3_sr;
      store_chunk(o3 + int64_t(ha) * p.o3_sh + d0, ra);
      store_chunk(o3 + int64_t(hb) * p.o3_sh + d0, rb);
    }
  }
}

template <typename T>
__global__ void __launch_bounds__(256) rope_givens_bwd_vec_kernel(const RopeBwdParams p) {
  using E = Elem<T>;
  constexpr int EPC = 16 / sizeof(T);
  constexpr int kMaxPairChunks = 2048;  // LDS slots for d theta partials (kRopeRows * H/2 * D/EPC)
  __shared__ float dth[kMaxPairChunks];
  __shared__ __align__(16) float tc[kRopeRows * kRopeMaxHalf], ts[kRopeRows * kRopeMaxHalf];
  __shared__ float gc[kRopeMaxPairs], gs[kRopeMaxPairs], gce[kRopeMaxPairs], gse[kRopeMaxPairs];
  const int HD = p.H * p.D, half = p.D / 2;
  const int npair = p.H / 2, cpg = p.D / EPC;   // chunks per head
  const int ur = p.H * (half / EPC);
  const int ug = npair * cpg;
  const int upr = ur + ug;
  const int rows = p.B * p.T;
  const int row0 = blockIdx.x * kRopeRows;
  rope_tables_lds<T>(p.inv_freq, p.theta, p.pos0, row0, p.T, half, npair, tc, ts, gc, gs, gce, gse);
  for (int u = threadIdx.x; u < kRopeRows * upr; u += blockDim.x) {
    const int rl = u / upr, k = u % upr;
    const int row = row0 + rl;
    if (row >= rows) break;
    const int b = row / p.T, t = row % p.T;
    T* dx = reinterpret_cast<T*>(p.dqkv) + int64_t(b) * p.dq_sb + int64_t(t) * p.dq_sr;
    if (k < ur) {
      const int hd = k / (half / EPC), k0 = (k % (half / EPC)) * EPC;
      const float* cs = tc + rl * half + k0;
      // transposed rotation: dx_k = d_k c + d_{k+h} s, dx_{k+h} = d_{k+h} c - d_k s
      float msn[EPC];
#pragma unroll
      for (int e = 0; e < EPC; ++e) msn[e] = -ts[rl * half + k0 + e];
      const T* g1 = reinterpret_cast<const T*>(p.g1) + int64_t(b) * p.g1_sb + int64_t(hd) * p.g1_sh + int64_t(t) * p.g1_sr;
      const T* g2 = reinterpret_cast<const T*>(p.g2) + int64_t(b) * p.g2_sb + int64_t(hd) * p.g2_sh + int64_t(t) * p.g2_sr;
      rope_chunk_fwd<T>(g1, dx + hd * p.D, half, k0, cs, msn);
      rope_chunk_fwd<T>(g2, dx + HD + hd * p.D, half, k0, cs, msn);
    } else {
      const int kg = k - ur;
      const int pr = kg / cpg, d0 = (kg % cpg) * EPC;
      int ha, hb;
      if (p.parity == 0) {
        ha = 2 * pr;
        hb = 2 * pr + 1;
      } else {
        ha = 2 * pr + 1;
        hb = (2 * pr + 2) % p.H;
      }
      const T* g3 = reinterpret_cast<const T*>(p.g3) + int64_t(b) * p.g3_sb + int64_t(t) * p.g3_sr;
      const Chunk ga = load_chunk(g3 + int64_t(ha) * p.g3_sh + d0), gb = load_chunk(g3 + int64_t(hb) * p.g3_sh + d0);
      Chunk ra = ga, rb = gb;
      if (p.theta) {
        const float c = gce[pr], sn = gse[pr];      // exact: the derivative of the unrounded function
        const float cr = gc[pr], sr = gs[pr];       // rounded: the rotation that was applied
        const T* xi = reinterpret_cast<const T*>(p.qkv) + int64_t(b) * p.qkv_sb + int64_t(t) * p.qkv_sr + 2 * HD;
        const Chunk xa = load_chunk(xi + ha * p.D + d0), xb = load_chunk(xi + hb * p.D + d0);
        const T* ega = reinterpret_cast<const T*>(&ga);
        const T* egb = reinterpret_cast<const T*>(&gb);
        const T* exa = reinterpret_cast<const T*>(&xa);
        const T* exb = reinterpret_cast<const T*>(&xb);
        T* oa = reinterpret_cast<T*>(&ra);
        T* ob = reinterpret_cast<T*>(&rb);
        float acc = 0.f;
#pragma unroll
        for (int e = 0; e < EPC; ++e) {
          const float a = E::to_f(exa[e]), bb = E::to_f(exb[e]);
          const float da = E::to_f(ega[e]), db = E::to_f(egb[e]);
          oa[e] = E::from_f(cr * da + sr * db);
          ob[e] = E::from_f(cr * db - sr * da);
          acc += da * (-sn * a - c * bb) + db * (c * a - sn * bb);
        }
        dth[(rl * npair + pr) * cpg + kg % cpg] = acc;
      }
      store_chunk(dx + 2 * HD + ha * p.D + d0, ra);
      store_chunk(dx + 2 * HD + hb * p.D + d0, rb);
    }
  }
  if (!p.theta) return;
  __syncthreads();
  // per pair: fixed-order sum over the block's rows and the head's chunks (one partial per block)
  for (int pr = threadIdx.x; pr < npair; pr += blockDim.x) {
    float acc = 0.f;
    for (int rl = 0; rl < kRopeRows; ++rl) {
      if (row0 + rl >= rows) break;
      for (int c = 0; c < cpg; ++c) acc += dth[(rl * npair + pr) * cpg + c];
    }
    p.partial[int64_t(blockIdx.x) * npair + pr] = acc;
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
  p.B = a->B; p.T = a->T; p.H = a->H; p.D = a->D; p.pos0 = a->pos0; p.parity = a->layer_parity & 1;
  const int rows = a->B * a->T;
  const int epc = a->dtype == MOTE_BF16 ? 8 : 4;
  const bool vec = (a->D / 2) % epc == 0 && a->D / 2 <= kRopeMaxHalf && a->H / 2 <= kRopeMaxPairs && aligned16(a);
  const int vblocks = (rows + kRopeRows - 1) / kRopeRows;
  if (a->dtype == MOTE_BF16) {
    if (vec) hipLaunchKernelGGL(rope_givens_fwd_vec_kernel<bf16_t>, dim3(vblocks), dim3(256), 0, stream, p);
    else hipLaunchKernelGGL(rope_givens_fwd_kernel<bf16_t>, dim3(rows), dim3(256), 0, stream, p);
  } else {
    if (vec) hipLaunchKernelGGL(rope_givens_fwd_vec_kernel<float>, dim3(vblocks), dim3(256), 0, stream, p);
    else hipLaunchKernelGGL(rope_givens_fwd_kernel<float>, dim3(rows), dim3(256), 0, stream, p);
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
  p.g1 = a->dp1.data; p.g1_sb = a->dp1.stride_b; p.g1_sh = a->dp1.stride_h; p.g1_sr = a->dp1.stride_r;
  p.g2 = a->dp2.data; p.g2_sb = a->dp2.stride_b; p.g2_sh = a->dp2.stride_h; p.g2_sr = a->dp2.stride_r;
  p.g3 = a->dinfo.data; p.g3_sb = a->dinfo.stride_b; p.g3_sh = a->dinfo.stride_h; p.g3_sr = a->dinfo.stride_r;
  p.dqkv = a->dqkv; p.dq_sb = a->dqkv_sb; p.dq_sr = a->dqkv_sr;
  p.inv_freq = a->inv_freq; p.theta = a->theta;
  p.partial = reinterpret_cast<float*>(a->workspace);
  p.B = a->B; p.T = a->T; p.H = a->H; p.D = a->D; p.pos0 = a->pos0; p.parity = a->layer_parity & 1;
  const int rows = a->B * a->T;
  const int epc = a->dtype == MOTE_BF16 ? 8 : 4;
  const bool vec = (a->D / 2) % epc == 0 && a->D / 2 <= kRopeMaxHalf && a->H / 2 <= kRopeMaxPairs &&
                   aligned16_bwd(a) && kRopeRows * (a->H / 2) * (a->D / epc) <= 2048;
  const int vblocks = (rows + kRopeRows - 1) / kRopeRows;
  if (a->dtype == MOTE_BF16) {
    if (vec) hipLaunchKernelGGL(rope_givens_bwd_vec_kernel<bf16_t>, dim3(vblocks), dim3(256), 0, stream, p);
    else hipLaunchKernelGGL(rope_givens_bwd_kernel<bf16_t>, dim3(rows), dim3(256), 0, stream, p);
  } else {
    if (vec) hipLaunchKernelGGL(rope_givens_bwd_vec_kernel<float>, dim3(vblocks), dim3(256), 0, stream, p);
    else hipLaunchKernelGGL(rope_givens_bwd_kernel<float>, dim3(rows), dim3(256), 0, stream, p);
  }
  rc = check_launch("rope_givens_bwd");
  if (rc || !a->theta) return rc;
  const int nparts = vec ? vblocks : rows;  // the vectorised kernel leaves one partial per block
  hipLaunchKernelGGL(sum_partials_kernel, dim3((a->H / 2 + 3) / 4), dim3(256), 0, stream, p.partial, nparts, a->H / 2,
                     a->dtheta);
  return check_launch("rope_givens_bwd/sum");
}

}  // namespace mote
