// One decode step of one Relation layer (mote/infer/graph.py:151-187), one launch.
//
// Grid: nsplit x (B*H) workgroups, block id = split * (B*H) + head index, so with B*H a multiple
// of 8 every split of one (sequence, head) runs on the same XCD (ids go round-robin over the 8 XCDs)
// and the merge reads partials from its own L2. Every split reads a contiguous range of the past
// rows [0, S) of its head:
//   phase 1  U_j = <q, P2_j> / sqrt(D) for its rows (4 lanes per row, 16-byte loads), exchange
//            score SiLU(U_j) in log2 units kept in LDS;
//   phase 2  the workgroup max, p_j = 2^(e_j - max), z += p_j I~_j, l += p_j.
// Each split writes (max, l, z[D]) to the workspace; the last split of a head to arrive (counter in
// the workspace, device-scope fences) merges them, computes the Self score from the new row,
// g = sigmoid(LSE - lam ln(S+1) - S_self) and Y = (1-g) I~_S + g z/l, and appends the new P2 / I~
// row at S. The merge resets the counter, so the workspace is ready for the next call and the
// launch can sit in a HIP graph. With MOTE_DECODE_ADVANCE the last head to finish adds 1 to every
// S[b] once all workgroups have read it.
//
// The query is RoPE'd at S and rounded to the cache dtype (graph.py:158-172) by every workgroup; the
// new P2 row gets the same rotation and I~ the Givens rotation with its partner head's raw row.
// Bandwidth-bound by design: no MFMA, wavefront reductions only.
#include "common.hpp"
#include "params.hpp"

namespace mote {

struct DecParams {
  const float* lam;
  const float* inv_freq;
  const float* theta;
  int64_t* S;
  const void* p1;
  const void* p2;
  const void* info;
  int64_t in_sb;
  const void* kc; int64_t kc_sb, kc_sh, kc_sr;
  const void* vc; int64_t vc_sb, vc_sh, vc_sr;
  void* kc_w;  // writable aliases of the caches (append)
  void* vc_w;
  void* y;
  int64_t y_sb;
  float* g;
  float* part;        // [BH][nsplit][D + 2]  (max, l, z)
  unsigned* counter;  // [BH + 1], zero between calls
  int B, H, D, cap, parity, flags, nsplit;
  float scale, tau_inv;
};

constexpr int kDecRowsMax = 2048;  // rows one split may own (LDS scores)

template <typename T>
__device__ __forceinline__ float round_to(float x) {
  return Elem<T>::to_f(Elem<T>::from_f(x));
}

template <typename T, int DP>
__global__ void __launch_bounds__(256) relation_decode_kernel(const DecParams p) {
  using E = Elem<T>;
  constexpr int EPC = 16 / sizeof(T);
  __shared__ float sq[DP];
  __shared__ float sc[kDecRowsMax];
  __shared__ float red[4 * DP + 8];
  __shared__ float sred[8];
  __shared__ int s_last;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int BH = p.B * p.H;
  const int bh = blockIdx.x % BH;
  const int split = blockIdx.x / BH;
  const int b = bh / p.H, h = bh % p.H;
  const int D = p.D, half = D / 2;
  const int64_t S64 = p.S[b];
  const bool bad = S64 < 0 || S64 >= p.cap;
  const int S = bad ? 0 : int(S64);

  // query: RoPE at S, rounded to the cache dtype
  const T* q_raw = reinterpret_cast<const T*>(p.p1) + b * p.in_sb + h * D;
  if (tid < half) {
    const float x0 = E::to_f(q_raw[tid]), x1 = E::to_f(q_raw[tid + half]);
    float o0 = x0, o1 = x1;
    if (p.inv_freq) {
      float sn, cs;
      sincosf((float)S * p.inv_freq[tid], &sn, &cs);
      cs = round_to<T>(cs);
      sn = round_to<T>(sn);
      o0 = x0 * cs - x1 * sn;
      o1 = x1 * cs + x0 * sn;
    }
    sq[tid] = round_to<T>(o0);
    sq[tid + half] = round_to<T>(o1);
  }
  for (int d = D + tid; d < DP; d += 256) sq[d] = 0.f;
  __syncthreads();

  // rows of this split
  const int chunk = (S + p.nsplit - 1) / p.nsplit;
  const int r0 = min(S, split * chunk);
  const int r1 = min(S, r0 + chunk);
  const int nrows = r1 - r0;
  const T* kbase = reinterpret_cast<const T*>(p.kc) + b * p.kc_sb + h * p.kc_sh;
  const T* vbase = reinterpret_cast<const T*>(p.vc) + b * p.vc_sb + h * p.vc_sh;
  const int rr = lane >> 2, c = lane & 3;
  const int nch = D / EPC;  // 16-byte chunks per row
  const float c2 = p.scale * kLog2e;

  // phase 1: exchange scores
  for (int base = 0; base < nrows; base += 64) {
    const int ri = base + wave * 16 + rr;
    float dot = 0.f;
    if (ri < nrows) {
      const T* row = kbase + int64_t(r0 + ri) * p.kc_sr;
      for (int k = c; k < nch; k += 4) {
        const Chunk ch = load_chunk(row + k * EPC);
        const T* e = reinterpret_cast<const T*>(&ch);
#pragma unroll
        for (int j = 0; j < EPC; ++j) dot = fmaf(E::to_f(e[j]), sq[k * EPC + j], dot);
      }
    }
    dot += __shfl_xor(dot, 1, 64);
    dot += __shfl_xor(dot, 2, 64);
    if (ri < nrows && c == 0) {
      const float u2 = dot * c2;
      sc[ri] = u2 * frcp(1.0f + fexp2(-u2));
    }
  }
  __syncthreads();
  // workgroup max
  float mx = kNegInf;
  for (int i = tid; i < nrows; i += 256) mx = fmaxf(mx, sc[i]);
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) mx = fmaxf(mx, __shfl_xor(mx, m, 64));
  if (lane == 0) sred[wave] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(sred[0], sred[1]), fmaxf(sred[2], sred[3]));
  const float msafe = mx == kNegInf ? 0.f : mx;

  // phase 2: z = sum p I~, l = sum p   (lane owns chunks c, c+4, ... of its rows)
  constexpr int MAXC = (DP / EPC + 3) / 4;  // chunks per lane
  float z[MAXC][EPC];
#pragma unroll
  for (int k = 0; k < MAXC; ++k)
#pragma unroll
    for (int j = 0; j < EPC; ++j) z[k][j] = 0.f;
  float l = 0.f;
  for (int base = 0; base < nrows; base += 64) {
    const int ri = base + wave * 16 + rr;
    if (ri < nrows) {
      const float pr = fexp2(sc[ri] - msafe);
      if (c == 0) l += pr;
      const T* row = vbase + int64_t(r0 + ri) * p.vc_sr;
#pragma unroll
      for (int k = 0; k < MAXC; ++k) {
        const int kc = c + 4 * k;
        if (kc < nch) {
          const Chunk ch = load_chunk(row + kc * EPC);
          const T* e = reinterpret_cast<const T*>(&ch);
#pragma unroll
          for (int j = 0; j < EPC; ++j) z[k][j] = fmaf(pr, E::to_f(e[j]), z[k][j]);
        }
      }
    }
  }
  // reduce over the 16 row groups of the wave (lanes with equal c)
#pragma unroll
  for (int m = 4; m <= 32; m <<= 1) {
    l += __shfl_xor(l, m, 64);
#pragma unroll
    for (int k = 0; k < MAXC; ++k)
#pragma unroll
      for (int j = 0; j < EPC; ++j) z[k][j] += __shfl_xor(z[k][j], m, 64);
  }
  if (rr == 0) {
#pragma unroll
    for (int k = 0; k < MAXC; ++k) {
      const int kc = c + 4 * k;
      if (kc < nch)
#pragma unroll
        for (int j = 0; j < EPC; ++j) red[wave * DP + kc * EPC + j] = z[k][j];
    }
    if (c == 0) red[4 * DP + wave] = l;
  }
  __syncthreads();
  float* part = p.part + (int64_t(bh) * p.nsplit + split) * (D + 2);
  for (int d = tid; d < D; d += 256) part[2 + d] = red[d] + red[DP + d] + red[2 * DP + d] + red[3 * DP + d];
  if (tid == 0) {
    part[0] = nrows > 0 ? mx : kNegInf;
    part[1] = red[4 * DP] + red[4 * DP + 1] + red[4 * DP + 2] + red[4 * DP + 3];
  }

  // ---- the last split of this head merges ----
  __threadfence();
  __syncthreads();
  if (tid == 0) s_last = atomicAdd(&p.counter[bh], 1u) == unsigned(p.nsplit - 1);
  __syncthreads();
  if (!s_last) return;
  __threadfence();
  const float* pb = p.part + int64_t(bh) * p.nsplit * (D + 2);
  float M = kNegInf;
  for (int s = 0; s < p.nsplit; ++s) M = fmaxf(M, pb[s * (D + 2)]);
  const float Ms = M == kNegInf ? 0.f : M;
  float L = 0.f;
  for (int s = 0; s < p.nsplit; ++s) {
    const float ms = pb[s * (D + 2)];
    const float ls = pb[s * (D + 2) + 1];
    if (ls > 0.f) L += ls * fexp2(ms - Ms);
  }
  // new rows: RoPE'd P2 (sq-style, into red[0..D)) and Givens'd I~ (red[DP..DP+D))
  const T* k_raw = reinterpret_cast<const T*>(p.p2) + b * p.in_sb + h * D;
  const T* i_raw = reinterpret_cast<const T*>(p.info) + b * p.in_sb + h * D;
  if (tid < half) {
    const float x0 = E::to_f(k_raw[tid]), x1 = E::to_f(k_raw[tid + half]);
    float o0 = x0, o1 = x1;
    if (p.inv_freq) {
      float sn, cs;
      sincosf((float)S * p.inv_freq[tid], &sn, &cs);
      cs = round_to<T>(cs);
      sn = round_to<T>(sn);
      o0 = x0 * cs - x1 * sn;
      o1 = x1 * cs + x0 * sn;
    }
    red[tid] = round_to<T>(o0);
    red[tid + half] = round_to<T>(o1);
  }
  if (tid < D) {
    const float self = E::to_f(i_raw[tid]);
    float out = self;
    if (p.theta) {
      int pair, other;
      bool first;
      if (p.parity == 0) {
        pair = h >> 1;
        first = (h & 1) == 0;
        other = first ? h + 1 : h - 1;
      } else if (h & 1) {
        first = true;
        pair = h >> 1;
        other = (h + 1) % p.H;
      } else {
        first = false;
        other = (h + p.H - 1) % p.H;
        pair = other >> 1;
      }
      float sn, cs;
      sincosf(p.theta[pair], &sn, &cs);
      cs = round_to<T>(cs);
      sn = round_to<T>(sn);
      const float oth = E::to_f(reinterpret_cast<const T*>(p.info)[b * p.in_sb + other * D + tid]);
      out = first ? (cs * self - sn * oth) : (sn * oth + cs * self);
    }
    red[DP + tid] = round_to<T>(out);
  }
  __syncthreads();
  // Self score U_SS = <q, P2_S> / sqrt(D)
  float u = 0.f;
  for (int d = tid; d < D; d += 256) u = fmaf(sq[d], red[d], u);
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) u += __shfl_xor(u, m, 64);
  if (lane == 0) sred[4 + wave] = u;
  __syncthreads();
  u = (sred[4] + sred[5] + sred[6] + sred[7]) * p.scale;
  const float sself = sigmoid_acc(u * p.tau_inv);
  const bool has = L > 0.f;
  const float lse = has ? (Ms + __log2f(L)) * kLn2 : kNegInf;
  const float gate = has ? sigmoid_acc(lse - (*p.lam) * logf((float)S + 1.0f) - sself) : 0.f;
  const float invL = has ? 1.0f / L : 0.f;
  T* y = reinterpret_cast<T*>(p.y) + b * p.y_sb + h * D;
  for (int d = tid; d < D; d += 256) {
    float zsum = 0.f;
    for (int s = 0; s < p.nsplit; ++s) {
      const float ls = pb[s * (D + 2) + 1];
      if (ls > 0.f) zsum += pb[s * (D + 2) + 2 + d] *
                            fexp2(pb[s * (D + 2)] - Ms);
    }
    const float yv = (1.0f - gate) * red[DP + d] + gate * zsum * invL;
    y[d] = E::from_f(bad ? __builtin_nanf("") : yv);
    if (!bad) {
      reinterpret_cast<T*>(p.kc_w)[b * p.kc_sb + h * p.kc_sh + int64_t(S) * p.kc_sr + d] = E::from_f(red[d]);
      reinterpret_cast<T*>(p.vc_w)[b * p.vc_sb + h * p.vc_sh + int64_t(S) * p.vc_sr + d] = E::from_f(red[DP + d]);
    }
  }
  if (tid == 0) {
    p.g[bh] = bad ? __builtin_nanf("") : gate;
    atomicExch(&p.counter[bh], 0u);
    if (p.flags & MOTE_DECODE_ADVANCE) {
      __threadfence();
      if (atomicAdd(&p.counter[BH], 1u) == unsigned(BH - 1)) {
        for (int bb = 0; bb < p.B; ++bb) atomicAdd(reinterpret_cast<unsigned long long*>(&p.S[bb]), 1ull);
        atomicExch(&p.counter[BH], 0u);
      }
    }
  }
}

static int decode_nsplit(const mote_relation_decode_args* a) {
  const int BH = a->B * a->H;
  int ns = (512 + BH - 1) / BH;
  ns = ns < 1 ? 1 : (ns > 64 ? 64 : ns);
  const int need = (a->capacity + kDecRowsMax - 1) / kDecRowsMax;
  return ns < need ? need : ns;
}

size_t decode_workspace_bytes(const mote_relation_decode_args* a) {
  const size_t BH = size_t(a->B) * a->H;
  const size_t counters = (BH + 1) * sizeof(unsigned);
  const size_t coff = (counters + 255) & ~size_t(255);
  return coff + BH * size_t(decode_nsplit(a)) * size_t(a->D + 2) * sizeof(float);
}

int launch_decode(const mote_relation_decode_args* a, hipStream_t stream) {
  if (!a) return set_error(MOTE_ERR_ARGUMENT, "relation_decode: null args");
  if (a->dtype != MOTE_F32 && a->dtype != MOTE_BF16) return set_error(MOTE_ERR_ARGUMENT, "relation_decode: bad dtype %d", a->dtype);
  if (a->D <= 0 || a->D > 128 || a->D % 8 != 0)
    return set_error(MOTE_ERR_SHAPE, "relation_decode: head dim %d unsupported (need 8 <= D <= 128, D %% 8 == 0)", a->D);
  if (a->B <= 0 || a->H <= 0 || a->H % 2 || a->capacity <= 0) return set_error(MOTE_ERR_SHAPE, "relation_decode: bad sizes");
  if (!a->lam || !a->S || !a->p1 || !a->p2 || !a->info || !a->cache_p2.data || !a->cache_info.data || !a->y || !a->g)
    return set_error(MOTE_ERR_ARGUMENT, "relation_decode: null pointer");
  if (!a->workspace || a->workspace_bytes < decode_workspace_bytes(a))
    return set_error(MOTE_ERR_WORKSPACE, "relation_decode: workspace of %zu bytes, %zu needed", a->workspace_bytes,
                     decode_workspace_bytes(a));
  DecParams p;
  p.lam = a->lam; p.inv_freq = a->inv_freq; p.theta = a->theta; p.S = a->S;
  p.p1 = a->p1; p.p2 = a->p2; p.info = a->info; p.in_sb = a->in_sb;
  p.kc = a->cache_p2.data; p.kc_sb = a->cache_p2.stride_b; p.kc_sh = a->cache_p2.stride_h; p.kc_sr = a->cache_p2.stride_r;
  p.vc = a->cache_info.data; p.vc_sb = a->cache_info.stride_b; p.vc_sh = a->cache_info.stride_h; p.vc_sr = a->cache_info.stride_r;
  p.kc_w = a->cache_p2.data; p.vc_w = a->cache_info.data;
  p.y = a->y; p.y_sb = a->y_sb; p.g = a->g;
  const size_t BH = size_t(a->B) * a->H;
  const size_t coff = ((BH + 1) * sizeof(unsigned) + 255) & ~size_t(255);
  p.counter = reinterpret_cast<unsigned*>(a->workspace);
  p.part = reinterpret_cast<float*>(reinterpret_cast<char*>(a->workspace) + coff);
  p.B = a->B; p.H = a->H; p.D = a->D; p.cap = a->capacity; p.parity = a->layer_parity & 1; p.flags = a->flags;
  p.nsplit = decode_nsplit(a);
  p.scale = 1.0f / sqrtf((float)a->D);
  p.tau_inv = 1.0f / a->tau_s;
  const int grid = int(BH) * p.nsplit;
  const int DP = padded_dim(a->D);
  if (a->dtype == MOTE_BF16) {
    switch (DP) {
      case 32: hipLaunchKernelGGL((relation_decode_kernel<bf16_t, 32>), dim3(grid), dim3(256), 0, stream, p); break;
      case 64: hipLaunchKernelGGL((relation_decode_kernel<bf16_t, 64>), dim3(grid), dim3(256), 0, stream, p); break;
      case 96: hipLaunchKernelGGL((relation_decode_kernel<bf16_t, 96>), dim3(grid), dim3(256), 0, stream, p); break;
      default: hipLaunchKernelGGL((relation_decode_kernel<bf16_t, 128>), dim3(grid), dim3(256), 0, stream, p); break;
    }
  } else {
    switch (DP) {
      case 32: hipLaunchKernelGGL((relation_decode_kernel<float, 32>), dim3(grid), dim3(256), 0, stream, p); break;
      case 64: hipLaunchKernelGGL((relation_decode_kernel<float, 64>), dim3(grid), dim3(256), 0, stream, p); break;
      case 96: hipLaunchKernelGGL((relation_decode_kernel<float, 96>), dim3(grid), dim3(256), 0, stream, p); break;
      default: hipLaunchKernelGGL((relation_decode_kernel<float, 128>), dim3(grid), dim3(256), 0, stream, p); break;
    }
  }
  return check_launch("relation_decode");
}

}  // namespace mote
