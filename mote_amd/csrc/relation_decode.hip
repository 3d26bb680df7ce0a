// One decode step of one Relation layer (mote/infer/graph.py:151-187), one launch.
//
// Grid: nsplit x (B*H) workgroups, block id = split * (B*H) + head index. Split s owns the past rows
// [s*R, (s+1)*R) of its head, R = 64 * rows_mult (a host choice that keeps a few hundred workgroups
// in flight); the launch shape depends only on the cache capacity, so it can be captured in a HIP
// graph. Each workgroup (4 waves; a wave reads 16 rows per step, 4 lanes per row, 16-byte loads of
// P2 and I~ issued together with a one-step register prefetch) computes U_j = <q, P2_j> / sqrt(D),
// e_j = SiLU(U_j) in log2 units and an online softmax per row group (running max raised lazily, by
// more than 2^8 only), merges its row groups and waves, and publishes (max, l, z[D]).
//
// Publication without a device-scope fence (which on gfx950 writes back the XCD's whole L2): the
// partial goes out with agent-coherent stores, the wave waits for their completion, and one atomic
// add per workgroup counts the head's splits. Every split counts, rows or not, so the count never
// depends on S. The workgroup that brings the count to nsplit reads all partials back with
// agent-coherent loads and finishes the head: merge in a fixed order, the Self score from the new
// row, g = sigmoid(LSE - lam ln(S+1) - S_self), Y = (1-g) I~_S + g z/l, the append of the new P2 / I~
// row at S, and the reset of the counter. A second counter per sequence picks the last head to
// finish; with MOTE_DECODE_ADVANCE it adds 1 to S[b]: by then every workgroup of the sequence has
// read S[b]. Counters start at zero (the workspace is zeroed once) and every call leaves them zero.
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
  void* kc; int64_t kc_sb, kc_sh, kc_sr;
  void* vc; int64_t vc_sb, vc_sh, vc_sr;
  void* y;
  int64_t y_sb;
  float* g;
  float* part;        // [BH][nsplit][D + 2]  (max, l, z)
  int* cnt;           // [BH] splits published in this call (zero between calls)
  int* cnt_seq;       // [B] heads finished in this call (zero between calls)
  int B, H, D, cap, parity, flags, nsplit, rps;  // rps: rows per split
  float scale, tau_inv;
};

constexpr int kDecMaxSplits = 120;  // partials one merge holds in LDS (D <= 128: at most 62 KB)

__device__ __forceinline__ void store_coherent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_coherent(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <typename T>
__device__ __forceinline__ float round_to(float x) {
  return Elem<T>::to_f(Elem<T>::from_f(x));
}

// ------------------------------------------------------------------------------------------------
// finish of a head by the last of its workgroups: merge, epilogue, append
// ------------------------------------------------------------------------------------------------
template <typename T, int DP>
__device__ __forceinline__ void decode_finish(const DecParams& p, int bh, int64_t S64) {
  using E = Elem<T>;
  __shared__ float sq[DP];
  __shared__ float knew[DP];
  __shared__ float inew[DP];
  __shared__ float sred[4];
  __shared__ float sML[2];
  extern __shared__ float spart[];  // [nsplit][D + 2], then the split weights [nsplit]

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int b = bh / p.H, h = bh % p.H;
  const int D = p.D, half = D / 2;
  const int stride = D + 2;
  const bool bad = S64 < 0 || S64 >= p.cap;
  const int S = bad ? 0 : int(S64);
  const int nact = p.nsplit;
  float* wsp = spart + nact * stride;
  const float* pb = p.part + int64_t(bh) * p.nsplit * stride;
  for (int i = tid; i < nact * stride; i += 256) spart[i] = load_coherent(pb + i);
  // new rows: query and P2 RoPE'd at S, I~ Givens'd with its partner head's raw row
  const T* q_raw = reinterpret_cast<const T*>(p.p1) + b * p.in_sb + h * D;
  const T* k_raw = reinterpret_cast<const T*>(p.p2) + b * p.in_sb + h * D;
  const T* i_raw = reinterpret_cast<const T*>(p.info) + b * p.in_sb + h * D;
  if (tid < half) {
    float cs = 1.f, sn = 0.f;
    if (p.inv_freq) {
      sincosf((float)S * p.inv_freq[tid], &sn, &cs);
      cs = round_to<T>(cs);
      sn = round_to<T>(sn);
    }
    const float q0 = E::to_f(q_raw[tid]), q1 = E::to_f(q_raw[tid + half]);
    const float k0 = E::to_f(k_raw[tid]), k1 = E::to_f(k_raw[tid + half]);
    sq[tid] = round_to<T>(q0 * cs - q1 * sn);
    sq[tid + half] = round_to<T>(q1 * cs + q0 * sn);
    knew[tid] = round_to<T>(k0 * cs - k1 * sn);
    knew[tid + half] = round_to<T>(k1 * cs + k0 * sn);
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
    inew[tid] = round_to<T>(out);
  }
  __syncthreads();
  // split weights 2^(m_s - M) and L = sum_s l_s 2^(m_s - M): wave 0, lanes over splits (fixed order)
  if (wave == 0) {
    float mx = kNegInf;
    for (int s = lane; s < nact; s += 64) mx = fmaxf(mx, spart[s * stride]);
#pragma unroll
    for (int msk = 32; msk >= 1; msk >>= 1) mx = fmaxf(mx, __shfl_xor(mx, msk, 64));
    const float Ms = mx == kNegInf ? 0.f : mx;
    float ls = 0.f;
    for (int s = lane; s < nact; s += 64) {
      const float w = fexp2(spart[s * stride] - Ms);
      wsp[s] = w;
      ls += spart[s * stride + 1] * w;
    }
#pragma unroll
    for (int msk = 32; msk >= 1; msk >>= 1) ls += __shfl_xor(ls, msk, 64);
    if (lane == 0) {
      sML[0] = Ms;
      sML[1] = ls;
    }
  } else if (wave == 1) {
    // Self score U_SS = <q, P2_S> / sqrt(D)
    float u = 0.f;
    for (int d = lane; d < D; d += 64) u = fmaf(sq[d], knew[d], u);
#pragma unroll
    for (int msk = 32; msk >= 1; msk >>= 1) u += __shfl_xor(u, msk, 64);
    if (lane == 0) sred[0] = u;
  }
  __syncthreads();
  const float Ms = sML[0], L = sML[1];
  const float sself = sigmoid_acc(sred[0] * p.scale * p.tau_inv);
  const bool has = L > 0.f;
  const float lse = has ? (Ms + __log2f(L)) * kLn2 : kNegInf;
  const float gate = has ? sigmoid_acc(lse - (*p.lam) * logf((float)S + 1.0f) - sself) : 0.f;
  const float invL = has ? 1.0f / L : 0.f;
  T* y = reinterpret_cast<T*>(p.y) + b * p.y_sb + h * D;
  T* kw = reinterpret_cast<T*>(p.kc) + b * p.kc_sb + h * p.kc_sh + int64_t(S) * p.kc_sr;
  T* vw = reinterpret_cast<T*>(p.vc) + b * p.vc_sb + h * p.vc_sh + int64_t(S) * p.vc_sr;
  for (int d = tid; d < D; d += 256) {
    float zsum = 0.f;
#pragma unroll 8
    for (int s = 0; s < nact; ++s) zsum = fmaf(spart[s * stride + 2 + d], wsp[s], zsum);
    const float yv = (1.0f - gate) * inew[d] + gate * zsum * invL;
    y[d] = E::from_f(bad ? __builtin_nanf("") : yv);
    if (!bad) {
      kw[d] = E::from_f(knew[d]);
      vw[d] = E::from_f(inew[d]);
    }
  }
  if (tid == 0) {
    p.g[bh] = bad ? __builtin_nanf("") : gate;
    __hip_atomic_store(p.cnt + bh, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    // the last head of the sequence: every workgroup of the sequence has read S[b] by now
    const int before = __hip_atomic_fetch_add(p.cnt_seq + b, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (before == p.H - 1) {
      __hip_atomic_store(p.cnt_seq + b, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (p.flags & MOTE_DECODE_ADVANCE) p.S[b] = S64 + 1;
    }
  }
}

template <typename T, int DP>
__global__ void __launch_bounds__(256) relation_decode_kernel(const DecParams p) {
  using E = Elem<T>;
  constexpr int EPC = 16 / sizeof(T);
  constexpr int MAXC = (DP / EPC + 3) / 4;  // 16-byte chunks per lane (lane c owns chunks c, c+4, ...)
  __shared__ float sq[DP];
  __shared__ float red[4 * (DP + 2)];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int BH = p.B * p.H;
  const int bh = blockIdx.x % BH;
  const int split = blockIdx.x / BH;
  const int b = bh / p.H, h = bh % p.H;
  const int D = p.D, half = D / 2;
  const int64_t S64 = p.S[b];
  const bool bad = S64 < 0 || S64 >= p.cap;
  const int S = bad ? 0 : int(S64);
  // every split takes part (those at or past S publish an empty partial), so the count of published
  // splits never depends on S

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

  const int r0 = split * p.rps;
  const int r1 = min(S, r0 + p.rps);
  const T* kbase = reinterpret_cast<const T*>(p.kc) + b * p.kc_sb + h * p.kc_sh;
  const T* vbase = reinterpret_cast<const T*>(p.vc) + b * p.vc_sb + h * p.vc_sh;
  const int rr = lane >> 2, c = lane & 3;
  const int nch = D / EPC;
  const float c2 = p.scale * kLog2e;
  float qv[MAXC][EPC];
#pragma unroll
  for (int k = 0; k < MAXC; ++k)
#pragma unroll
    for (int j = 0; j < EPC; ++j) qv[k][j] = (c + 4 * k) < nch ? sq[(c + 4 * k) * EPC + j] : 0.f;

  float m = kNegInf, l = 0.f;
  float z[MAXC][EPC];
#pragma unroll
  for (int k = 0; k < MAXC; ++k)
#pragma unroll
    for (int j = 0; j < EPC; ++j) z[k][j] = 0.f;

  Chunk kr[MAXC], vr[MAXC];
  auto fetch = [&](int row) {
#pragma unroll
    for (int k = 0; k < MAXC; ++k) {
      const int kc = c + 4 * k;
      if (row < r1 && kc < nch) {
        kr[k] = load_chunk(kbase + int64_t(row) * p.kc_sr + kc * EPC);
        vr[k] = load_chunk(vbase + int64_t(row) * p.vc_sr + kc * EPC);
      } else {
        kr[k] = zero_chunk();
        vr[k] = zero_chunk();
      }
    }
  };
  int row = r0 + wave * 16 + rr;
  fetch(row);
  for (int base = r0; base < r1; base += 64) {
    Chunk kc_[MAXC], vc_[MAXC];
#pragma unroll
    for (int k = 0; k < MAXC; ++k) {
      kc_[k] = kr[k];
      vc_[k] = vr[k];
    }
    const int cur = row;
    row += 64;
    if (base + 64 < r1) fetch(row);  // prefetch the next step while this one computes
    float dot = 0.f;
#pragma unroll
    for (int k = 0; k < MAXC; ++k) {
      const T* e = reinterpret_cast<const T*>(&kc_[k]);
#pragma unroll
      for (int j = 0; j < EPC; ++j) dot = fmaf(E::to_f(e[j]), qv[k][j], dot);
    }
    dot += __shfl_xor(dot, 1, 64);
    dot += __shfl_xor(dot, 2, 64);
    if (cur < r1) {
      const float u2 = dot * c2;
      const float ev = u2 * frcp(1.0f + fexp2(-u2));
      if (ev > m + kRescale) {
        const float alpha = fexp2(m - ev);  // 0 on the first row
        l *= alpha;
#pragma unroll
        for (int k = 0; k < MAXC; ++k)
#pragma unroll
          for (int j = 0; j < EPC; ++j) z[k][j] *= alpha;
        m = ev;
      }
      const float pr = fexp2(ev - m);
      l += pr;
#pragma unroll
      for (int k = 0; k < MAXC; ++k) {
        const T* e = reinterpret_cast<const T*>(&vc_[k]);
#pragma unroll
        for (int j = 0; j < EPC; ++j) z[k][j] = fmaf(pr, E::to_f(e[j]), z[k][j]);
      }
    }
  }
  // merge the 16 row groups of the wave (lanes with equal c hold the same chunks)
#pragma unroll
  for (int msk = 4; msk <= 32; msk <<= 1) {
    const float mo = __shfl_xor(m, msk, 64);
    const float lo = __shfl_xor(l, msk, 64);
    const float mn = fmaxf(m, mo);
    const float ms = mn == kNegInf ? 0.f : mn;
    const float a = fexp2(m - ms), ao = fexp2(mo - ms);
    l = l * a + lo * ao;
#pragma unroll
    for (int k = 0; k < MAXC; ++k)
#pragma unroll
      for (int j = 0; j < EPC; ++j) z[k][j] = z[k][j] * a + __shfl_xor(z[k][j], msk, 64) * ao;
    m = mn;
  }
  if (rr == 0) {
#pragma unroll
    for (int k = 0; k < MAXC; ++k) {
      const int kc = c + 4 * k;
      if (kc < nch)
#pragma unroll
        for (int j = 0; j < EPC; ++j) red[wave * (DP + 2) + 2 + kc * EPC + j] = z[k][j];
    }
    if (c == 0) {
      red[wave * (DP + 2)] = m;
      red[wave * (DP + 2) + 1] = l;
    }
  }
  __syncthreads();
  // merge the 4 waves -> this split's partial
  {
    float mw[4];
    float M = kNegInf;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      mw[w] = red[w * (DP + 2)];
      M = fmaxf(M, mw[w]);
    }
    const float Ms = M == kNegInf ? 0.f : M;
    float* part = p.part + (int64_t(bh) * p.nsplit + split) * (D + 2);
    for (int d = tid; d < D; d += 256) {
      float zs = 0.f;
#pragma unroll
      for (int w = 0; w < 4; ++w) zs += red[w * (DP + 2) + 2 + d] * fexp2(mw[w] - Ms);
      store_coherent(part + 2 + d, zs);
    }
    if (tid == 0) {
      float L = 0.f;
#pragma unroll
      for (int w = 0; w < 4; ++w) L += red[w * (DP + 2) + 1] * fexp2(mw[w] - Ms);
      store_coherent(part, M);
      store_coherent(part + 1, L);
    }
  }
  // publish: every wave's coherent stores complete, then one count per workgroup
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  __shared__ int s_last;
  if (tid == 0) {
    const int before = __hip_atomic_fetch_add(p.cnt + bh, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = before == p.nsplit - 1;
  }
  __syncthreads();
  if (!s_last) return;
  decode_finish<T, DP>(p, bh, S64);
}

// rows per split: a multiple of 64 chosen so that about 320 workgroups cover a full cache
static void decode_shape(const mote_relation_decode_args* a, int& rps, int& nsplit) {
  const int64_t BH = int64_t(a->B) * a->H;
  int64_t mult = (BH * ((a->capacity + 63) / 64) + 319) / 320;
  if (mult < 1) mult = 1;
  rps = int(64 * mult);
  nsplit = (a->capacity + rps - 1) / rps;
  while (nsplit > kDecMaxSplits) {
    rps += 64;
    nsplit = (a->capacity + rps - 1) / rps;
  }
}

struct DecWs {
  size_t part, cnt, cnt_seq, total;
};
static DecWs decode_ws(const mote_relation_decode_args* a) {
  int rps, nsplit;
  decode_shape(a, rps, nsplit);
  const size_t BH = size_t(a->B) * a->H;
  DecWs w;
  w.part = 0;
  w.cnt = (BH * size_t(nsplit) * size_t(a->D + 2) * sizeof(float) + 255) & ~size_t(255);
  w.cnt_seq = w.cnt + ((BH * sizeof(int) + 255) & ~size_t(255));
  w.total = w.cnt_seq + ((size_t(a->B) * sizeof(int) + 255) & ~size_t(255));
  return w;
}

size_t decode_workspace_bytes(const mote_relation_decode_args* a) { return decode_ws(a).total; }

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
  p.y = a->y; p.y_sb = a->y_sb; p.g = a->g;
  const size_t BH = size_t(a->B) * a->H;
  decode_shape(a, p.rps, p.nsplit);
  const DecWs w = decode_ws(a);
  char* ws = reinterpret_cast<char*>(a->workspace);
  p.part = reinterpret_cast<float*>(ws + w.part);
  p.cnt = reinterpret_cast<int*>(ws + w.cnt);
  p.cnt_seq = reinterpret_cast<int*>(ws + w.cnt_seq);
  p.B = a->B; p.H = a->H; p.D = a->D; p.cap = a->capacity; p.parity = a->layer_parity & 1; p.flags = a->flags;
  p.scale = 1.0f / sqrtf((float)a->D);
  p.tau_inv = 1.0f / a->tau_s;
  const int grid = int(BH) * p.nsplit;
  const size_t shmem = size_t(p.nsplit) * (a->D + 3) * sizeof(float);
  const int DP = padded_dim(a->D);
#define MOTE_DEC_LAUNCH(T_, DP_)                                                                               \
  do {                                                                                                       \
    hipLaunchKernelGGL((relation_decode_kernel<T_, DP_>), dim3(grid), dim3(256), shmem, stream, p);          \
  } while (0)
  if (a->dtype == MOTE_BF16) {
    switch (DP) {
      case 32: MOTE_DEC_LAUNCH(bf16_t, 32); break;
      case 64: MOTE_DEC_LAUNCH(bf16_t, 64); break;
      case 96: MOTE_DEC_LAUNCH(bf16_t, 96); break;
      default: MOTE_DEC_LAUNCH(bf16_t, 128); break;
    }
  } else {
    switch (DP) {
      case 32: MOTE_DEC_LAUNCH(float, 32); break;
      case 64: MOTE_DEC_LAUNCH(float, 64); break;
      case 96: MOTE_DEC_LAUNCH(float, 96); break;
      default: MOTE_DEC_LAUNCH(float, 128); break;
    }
  }
#undef MOTE_DEC_LAUNCH
  return check_launch("relation_decode");
}

}  // namespace mote
