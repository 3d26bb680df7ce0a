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
// batch), then a fixed tree over the block: the order is fixed, so the result is reproducible.
__global__ void __launch_bounds__(256) sum_partials_kernel(const float* partial, int rows, int npair, float* out) {
  __shared__ float red[256];
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
  red[tid] = acc;
  __syncthreads();
  for (int w = 128; w >= 1; w >>= 1) {
    if (tid < w) red[tid] += red[tid + w];
    __syncthreads();
  }
  if (tid == 0) out[pr] = red[0];
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
// the RoPE factors of the block's rows go through LDS, and the only barrier waits for them.
// ------------------------------------------------------------------------------------------------
constexpr int kRopeNR = 4;
constexpr int kRopeMaxThreads = 1024;

// The RoPE factors of a block's nr rows, [nr][D/2] cos then sin in LDS, rounded to the element type
// as the reference casts its tables. Entry i = r D/2 + k goes to thread i mod blockDim: a sincos of
// a large angle (positions in the thousands) takes the long argument reduction, so the entries are
// spread over the whole block rather than left to D/2 threads. The inverse frequencies of a thread's
// first two entries (`inv2`) are loaded before the chunk loads, so the sincos runs while they arrive.
struct RopeInv {
  float v[2];
};
__device__ __forceinline__ RopeInv rope_inv(const float* inv_safe, int rope, int half) {
  RopeInv R;
  R.v[0] = inv_safe[(threadIdx.x % half) * rope];
  R.v[1] = inv_safe[((threadIdx.x + blockDim.x) % half) * rope];
  return R;
}
template <typename T>
__device__ __forceinline__ void rope_factors(const RopeInv& inv2, const float* inv_safe, int rope, int pos0, int row0,
                                             int nr, int nrow, int T_, int half, float* tc, float* ts) {
  int j = 0;
  for (int i = threadIdx.x; i < nr * half; i += blockDim.x, ++j) {
    const int r = i / half, k = i - r * half;
    const int t = (row0 + min(r, nrow - 1)) % T_;
    const float invk = j == 0 ? inv2.v[0] : j == 1 ? inv2.v[1] : inv_safe[k * rope];
    float sn, cs;
    sincosf((float)(pos0 + t) * invk, &sn, &cs);
    tc[i] = rope ? rnd<T>(cs) : 1.f;
    ts[i] = rope ? rnd<T>(sn) : 0.f;
  }
}

// A thread's rotation unit: tensor (0: p1, 1: p2, 2: I~), the two heads (one head for RoPE), the
// chunk k (RoPE: k < cph / 2, its partner k + cph / 2; Givens: the same chunk k < cph of both
// heads), the Givens pair, and the two chunks' positions in the [p1 | p2 | I~] row. Givens pairs
// (relation.py:150-174): even layers (0,1),(2,3)..., odd layers (1,2),...,(H-1,0); the first head of a
// pair gets c a - s b, the second s a + c b.
struct RopeUnit {
  int which, ha, hb, k, pair, ca, cb;
};
__device__ __forceinline__ RopeUnit rope_unit(int u, int H, int cph, int parity) {
  RopeUnit R;
  const int hch = cph / 2, ur = 2 * H * hch, cpt = H * cph;
  if (u < ur) {
    R.which = u / (H * hch);
    const int rem = u - R.which * H * hch;
    R.ha = R.hb = rem / hch;
    R.k = rem - R.ha * hch;
    R.pair = 0;
    R.ca = R.which * cpt + R.ha * cph + R.k;
    R.cb = R.ca + hch;
  } else {
    const int g = u - ur;
    R.which = 2;
    R.pair = g / cph;
    R.k = g - R.pair * cph;
    R.ha = parity == 0 ? 2 * R.pair : 2 * R.pair + 1;
    R.hb = parity == 0 ? 2 * R.pair + 1 : (2 * R.pair + 2) % H;
    R.ca = 2 * cpt + R.ha * cph + R.k;
    R.cb = 2 * cpt + R.hb * cph + R.k;
  }
  return R;
}

template <typename T>
__global__ void __launch_bounds__(kRopeMaxThreads) rope_givens_fwd_stream_kernel(const RopeParams p, int NS) {
  using E = Elem<T>;
  constexpr int EPC = 16 / sizeof(T);
  extern __shared__ float rope_tab[];  // [NS kRopeNR][D/2] cos, then sin
  const int tid = threadIdx.x;
  const int H = p.H, D = p.D, half = D / 2, npair = H / 2, cph = D / EPC, hch = cph / 2;
  const int U = 3 * H * cph / 2, rpb = NS * kRopeNR;
  const int rows = p.B * p.T;
  const int row0 = blockIdx.x * rpb;
  const int nrow = min(rpb, rows - row0);
  float* tc = rope_tab;
  float* ts = rope_tab + rpb * half;
  const bool act = tid < NS * U;
  const int slot = act ? tid / U : 0;
  const RopeUnit R = rope_unit(act ? tid - slot * U : 0, H, cph, p.parity);

  // table values first (indices by multiplication with the 0/1 flags: a select becomes a branch)
  const RopeInv inv2 = rope_inv(p.inv_safe, p.rope, half);
  const float th = p.theta_safe[min(R.pair, npair - 1) * p.givens];
  Chunk xa[kRopeNR], xb[kRopeNR];
  const T* q = reinterpret_cast<const T*>(p.qkv);
#pragma unroll
  for (int r = 0; r < kRopeNR; ++r) {
    const int row = row0 + min(NS * r + slot, nrow - 1), b = row / p.T, t = row - b * p.T;
    const T* base = q + int64_t(b) * p.qkv_sb + int64_t(t) * p.qkv_sr;
    xa[r] = load_chunk(base + R.ca * EPC);
    xb[r] = load_chunk(base + R.cb * EPC);
  }
  rope_factors<T>(inv2, p.inv_safe, p.rope, p.pos0, row0, rpb, nrow, p.T, half, tc, ts);
  float gsn, gcs;
  sincosf(th, &gsn, &gcs);
  const float gc = p.givens ? rnd<T>(gcs) : 1.f, gs = p.givens ? rnd<T>(gsn) : 0.f;
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
  T* oa = obase + int64_t(R.ha) * osh + R.k * EPC;
  T* ob = rope_part ? oa + hch * EPC : obase + int64_t(R.hb) * osh + R.k * EPC;
  const int a0 = R.k * EPC;  // RoPE factor index of the chunk's first element
#pragma unroll
  for (int r = 0; r < kRopeNR; ++r) {
    const int rr = NS * r + slot;
    if (rr >= nrow) break;
    const int row = row0 + rr, b = row / p.T, t = row - b * p.T;
    const T* ea = reinterpret_cast<const T*>(&xa[r]);
    const T* eb = reinterpret_cast<const T*>(&xb[r]);
    Chunk outa, outb;
    T* ya = reinterpret_cast<T*>(&outa);
    T* yb = reinterpret_cast<T*>(&outb);
#pragma unroll
    for (int e = 0; e < EPC; ++e) {
      const float C = rope_part ? tc[rr * half + a0 + e] : gc;
      const float S = rope_part ? ts[rr * half + a0 + e] : gs;
      const float va = E::to_f(ea[e]), vb = E::to_f(eb[e]);
      ya[e] = E::from_f(rot_round<T>(va, C, vb, -S));
      yb[e] = E::from_f(rot_round<T>(vb, C, va, S));
    }
    const int64_t off = int64_t(b) * osb + int64_t(t) * osr;
    store_chunk(oa + off, outa);
    store_chunk(ob + off, outb);
  }
}

template <typename T>
__global__ void __launch_bounds__(kRopeMaxThreads) rope_givens_bwd_stream_kernel(const RopeBwdParams p, int NS) {
  using E = Elem<T>;
  constexpr int EPC = 16 / sizeof(T);
  extern __shared__ float rope_tab[];  // [NS kRopeNR][D/2] cos, sin, then [threads] d theta
  const int tid = threadIdx.x;
  const int H = p.H, D = p.D, half = D / 2, npair = H / 2, cph = D / EPC, hch = cph / 2;
  const int U = 3 * H * cph / 2, rpb = NS * kRopeNR, ur = 2 * H * hch;
  const int rows = p.B * p.T;
  const int row0 = blockIdx.x * rpb;
  const int nrow = min(rpb, rows - row0);
  float* tc = rope_tab;
  float* ts = rope_tab + rpb * half;
  float* red = rope_tab + 2 * rpb * half;
  const bool act = tid < NS * U;
  const int slot = act ? tid / U : 0;
  const int u = act ? tid - slot * U : 0;
  const RopeUnit R = rope_unit(u, H, cph, p.parity);

  const RopeInv inv2 = rope_inv(p.inv_safe, p.rope, half);
  const float th = p.theta_safe[min(R.pair, npair - 1) * p.givens];
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
  const T* gpa = gb + int64_t(R.ha) * gsh + R.k * EPC;
  const T* gpb = R.which < 2 ? gpa + hch * EPC : gb + int64_t(R.hb) * gsh + R.k * EPC;
  // the pair's I~ inputs (for d theta); RoPE units load their head's I~ chunk instead, so that no
  // load sits under a lane condition
  const T* xq = reinterpret_cast<const T*>(p.qkv) + p.ioff + (R.k % cph) * EPC;
  Chunk g0[kRopeNR], g1[kRopeNR], x0[kRopeNR], x1[kRopeNR];
#pragma unroll
  for (int r = 0; r < kRopeNR; ++r) {
    const int row = row0 + min(NS * r + slot, nrow - 1), b = row / p.T, t = row - b * p.T;
    const int64_t go = int64_t(b) * gsb + int64_t(t) * gsr;
    g0[r] = load_chunk(gpa + go);
    g1[r] = load_chunk(gpb + go);
    const T* xr = xq + int64_t(b) * p.qkv_sb + int64_t(t) * p.qkv_sr;
    x0[r] = load_chunk(xr + R.ha * D);
    x1[r] = load_chunk(xr + R.hb * D);
  }
  rope_factors<T>(inv2, p.inv_safe, p.rope, p.pos0, row0, rpb, nrow, p.T, half, tc, ts);
  float gsn, gcs;
  sincosf(th, &gsn, &gcs);
  const float ce = p.givens ? gcs : 1.f, se = p.givens ? gsn : 0.f;                  // exact: the derivative
  const float cr = p.givens ? rnd<T>(gcs) : 1.f, sr = p.givens ? rnd<T>(gsn) : 0.f;  // applied rotation
  __syncthreads();

  // RoPE^T: dx_k = d_k c + d_{k+D/2} s, dx_{k+D/2} = d_{k+D/2} c - d_k s; Givens^T: da = c ga + s gb,
  // db = c gb - s ga
  const bool rope_part = R.which < 2;
  const bool dth_unit = act && !rope_part && p.givens;
  T* da_out = reinterpret_cast<T*>(p.dqkv) + R.ca * EPC;
  T* db_out = reinterpret_cast<T*>(p.dqkv) + R.cb * EPC;
  const int a0 = R.k * EPC;
  float acc = 0.f;
#pragma unroll
  for (int r = 0; r < kRopeNR; ++r) {
    const int rr = NS * r + slot;
    if (rr >= nrow) break;
    const int row = row0 + rr, b = row / p.T, t = row - b * p.T;
    const T* e0 = reinterpret_cast<const T*>(&g0[r]);
    const T* e1 = reinterpret_cast<const T*>(&g1[r]);
    Chunk outa, outb;
    T* ya = reinterpret_cast<T*>(&outa);
    T* yb = reinterpret_cast<T*>(&outb);
#pragma unroll
    for (int e = 0; e < EPC; ++e) {
      const float C = rope_part ? tc[rr * half + a0 + e] : cr;
      const float S = rope_part ? ts[rr * half + a0 + e] : sr;
      const float ga = E::to_f(e0[e]), gbv = E::to_f(e1[e]);
      ya[e] = E::from_f(ga * C + gbv * S);
      yb[e] = E::from_f(gbv * C + ga * -S);
    }
    if (act) {
      const int64_t off = int64_t(b) * p.dq_sb + int64_t(t) * p.dq_sr;
      store_chunk(da_out + off, outa);
      store_chunk(db_out + off, outb);
    }
    if (dth_unit) {
      // d theta of the pair: ga (-s a - c b) + gb (c a - s b), exact s, c
      const T* ea = reinterpret_cast<const T*>(&x0[r]);
      const T* eb = reinterpret_cast<const T*>(&x1[r]);
#pragma unroll
      for (int e = 0; e < EPC; ++e) {
        const float a = E::to_f(ea[e]), bb = E::to_f(eb[e]);
        const float da = E::to_f(e0[e]), db = E::to_f(e1[e]);
        acc += da * (-se * a - ce * bb) + db * (ce * a - se * bb);
      }
    }
  }
  if (!p.givens) return;
  // one partial per block and pair: the pair's units in a fixed order (slot, then chunk)
  red[tid] = dth_unit ? acc : 0.f;
  __syncthreads();
  for (int pr = tid; pr < npair; pr += blockDim.x) {
    float s2 = 0.f;
    for (int sl = 0; sl < NS; ++sl)
      for (int k = 0; k < cph; ++k) s2 += red[sl * U + ur + pr * cph + k];
    p.partial[int64_t(blockIdx.x) * npair + pr] = s2;
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
  return units <= kRopeMaxThreads;
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
    const int blocks = (rows + NS * kRopeNR - 1) / (NS * kRopeNR);
    const int threads = (NS * units + 63) / 64 * 64;
    const size_t lds = size_t(2) * NS * kRopeNR * (a->D / 2) * sizeof(float);
    if (a->dtype == MOTE_BF16)
      hipLaunchKernelGGL(rope_givens_fwd_stream_kernel<bf16_t>, dim3(blocks), dim3(threads), lds, stream, p, NS);
    else
      hipLaunchKernelGGL(rope_givens_fwd_stream_kernel<float>, dim3(blocks), dim3(threads), lds, stream, p, NS);
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
  const bool vec = stream_shape(a->H, a->D, epc, units, NS) && aligned16_bwd(a);
  const int blocks = vec ? (rows + NS * kRopeNR - 1) / (NS * kRopeNR) : rows;
  if (vec) {
    const int threads = (NS * units + 63) / 64 * 64;
    const size_t lds = (size_t(2) * NS * kRopeNR * (a->D / 2) + size_t(threads)) * sizeof(float);
    if (a->dtype == MOTE_BF16)
      hipLaunchKernelGGL(rope_givens_bwd_stream_kernel<bf16_t>, dim3(blocks), dim3(threads), lds, stream, p, NS);
    else
      hipLaunchKernelGGL(rope_givens_bwd_stream_kernel<float>, dim3(blocks), dim3(threads), lds, stream, p, NS);
  } else if (a->dtype == MOTE_BF16) {
    hipLaunchKernelGGL(rope_givens_bwd_kernel<bf16_t>, dim3(rows), dim3(256), 0, stream, p);
  } else {
    hipLaunchKernelGGL(rope_givens_bwd_kernel<float>, dim3(rows), dim3(256), 0, stream, p);
  }
  rc = check_launch("rope_givens_bwd");
  if (rc || !a->theta) return rc;
  const int nparts = blocks;  // one partial per block (the per-row kernel: one per row)
  hipLaunchKernelGGL(sum_partials_kernel, dim3(a->H / 2), dim3(256), 0, stream, p.partial, nparts, a->H / 2, a->dtheta);
  return check_launch("rope_givens_bwd/sum");
}

}  // namespace mote
