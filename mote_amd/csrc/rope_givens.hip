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
  // one block per pair; fixed-order strided sums, then a fixed tree
  __shared__ float red[256];
  const int pr = blockIdx.x;
  float acc = 0.f;
  for (int r = threadIdx.x; r < rows; r += 256) acc += partial[int64_t(r) * npair + pr];
  red[threadIdx.x] = acc;
  __syncthreads();
  for (int w = 128; w >= 1; w >>= 1) {
    if ((int)threadIdx.x < w) red[threadIdx.x] += red[threadIdx.x + w];
    __syncthreads();
  }
  if (threadIdx.x == 0) out[pr] = red[0];
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
  if (a->dtype == MOTE_BF16)
    hipLaunchKernelGGL(rope_givens_fwd_kernel<bf16_t>, dim3(rows), dim3(256), 0, stream, p);
  else
    hipLaunchKernelGGL(rope_givens_fwd_kernel<float>, dim3(rows), dim3(256), 0, stream, p);
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
  if (a->dtype == MOTE_BF16)
    hipLaunchKernelGGL(rope_givens_bwd_kernel<bf16_t>, dim3(rows), dim3(256), 0, stream, p);
  else
    hipLaunchKernelGGL(rope_givens_bwd_kernel<float>, dim3(rows), dim3(256), 0, stream, p);
  rc = check_launch("rope_givens_bwd");
  if (rc || !a->theta) return rc;
  hipLaunchKernelGGL(sum_partials_kernel, dim3(a->H / 2), dim3(256), 0, stream, p.partial, rows, a->H / 2, a->dtheta);
  return check_launch("rope_givens_bwd/sum");
}

}  // namespace mote
