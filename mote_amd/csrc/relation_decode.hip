// One decode step of one Relation layer (mote/infer/graph.py:151-187), one launch.
//
// Grid: nsplit x (B*H) workgroups, block id = split * (B*H) + head index; nsplit is a host choice
// from the shape only (about three workgroups per CU over the batch, no split shorter than 512 rows
// at full capacity), so the launch can be captured in a HIP graph. On the device each head's S past
// rows are cut into nsplit equal runs (multiples of the 64-row step) from S itself, so the splits
// stay balanced as S grows. Each workgroup (4 waves; a wave reads 16 rows per step, 4 lanes per row,
// 16-byte loads of P2 and I~, with a ring of four register sets keeping three steps of loads in
// flight) computes U_j = <q, P2_j> / sqrt(D), e_j = SiLU(U_j) in log2 units and an online softmax
// per row group (running max raised lazily, by more than 2^8 only), merges its row groups and waves,
// and publishes (max, l, z[D]).
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
#include <type_traits>

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
  int B, H, D, cap, parity, flags, nsplit;
  float scale, tau_inv;
};

constexpr int kDecMaxSplits = 120;  // partials one merge holds in LDS (D <= 128: at most 62 KB)
constexpr int kDecWaves = 4;  // waves per workgroup: 16 rows each per step (8 and 16 measured slower)
constexpr int kDecThreads = 64 * kDecWaves;

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
  for (int i = tid; i < nact * stride; i += kDecThreads) spart[i] = load_coherent(pb + i);
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
  for (int d = tid; d < D; d += kDecThreads) {
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
__global__ void __launch_bounds__(kDecThreads)
relation_decode_kernel(const DecParams p) {
  using E = Elem<T>;
  constexpr int EPC = 16 / sizeof(T);
  constexpr int MAXC = (DP / EPC + 3) / 4;  // 16-byte chunks per lane (lane c owns chunks c, c+4, ...)
  __shared__ float sq[DP];
  __shared__ float red[kDecWaves * (DP + 2)];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int BH = p.B * p.H;
  const int bh = blockIdx.x % BH;
  const int split = blockIdx.x / BH;
  const int b = bh / p.H, h = bh % p.H;
  const int D = p.D, half = D / 2;
  // Order of the prologue: the raw query loads, then the first NR - 1 cache steps, and only then the
  // position S (the split's rows do not depend on S, only where its valid rows end), the RoPE of the
  // query at S and the masks: the cache loads are in flight while S and the query arrive.
  const T* q_raw = reinterpret_cast<const T*>(p.p1) + b * p.in_sb + h * D;
  const int qi = min(tid, half - 1);
  const float x0 = E::to_f(q_raw[qi]), x1 = E::to_f(q_raw[qi + half]);

  // The head's S past rows are cut into nsplit equal runs (a multiple of the 64-row step) from S
  // itself, so every split carries the same load whatever S is; the grid depends only on the shape.
  const int64_t S64 = p.S[b];
  const bool bad = S64 < 0 || S64 >= p.cap;
  const int S = bad ? 0 : int(S64);
  const int rps = ((S + p.nsplit - 1) / p.nsplit + 63) & ~63;
  const int r0 = split * rps;
  const int rf = min(p.cap, r0 + rps);  // rows this split may load (the cache holds them all)
  const T* kbase = reinterpret_cast<const T*>(p.kc) + b * p.kc_sb + h * p.kc_sh;
  const T* vbase = reinterpret_cast<const T*>(p.vc) + b * p.vc_sb + h * p.vc_sh;
  const int rr = lane >> 2, c = lane & 3;
  const int nch = D / EPC;
  const float c2 = p.scale * kLog2e;

  // A ring of NR register sets, one 64-row step each (16 rows per wave, 4 lanes per row): the loads
  // of the next NR - 1 steps are in flight while a step computes, and the loop is unrolled by NR so
  // every set is named by a constant (a copy between sets would make the compiler wait for the
  // newest loads before issuing the next ones).
  constexpr int NR = 4;
  Chunk kr[NR][MAXC], vr[NR][MAXC];
  // Loads are unconditional (rows past the split and chunks past the head dim read a clamped, valid
  // address whose values the math ignores): a load under a lane condition would hide it from the
  // compiler's count of outstanding loads, and it would then wait for every one of them.
  auto fetch = [&](int row, auto u) {
    constexpr int U = decltype(u)::value;
    const int rc = max(0, min(row, rf - 1));
#pragma unroll
    for (int k = 0; k < MAXC; ++k) {
      const int kc = min(c + 4 * k, nch - 1);
      kr[U][k] = load_chunk(kbase + int64_t(rc) * p.kc_sr + kc * EPC);
      vr[U][k] = load_chunk(vbase + int64_t(rc) * p.vc_sr + kc * EPC);
    }
  };
  const int row0 = r0 + wave * 16 + rr;
  fetch(row0, std::integral_constant<int, 0>{});
  fetch(row0 + 16 * kDecWaves, std::integral_constant<int, 1>{});
  fetch(row0 + 32 * kDecWaves, std::integral_constant<int, 2>{});

  // every split takes part (those at or past S publish an empty partial), so the count of published
  // splits never depends on S
  // query: RoPE at S, rounded to the cache dtype
  if (tid < half) {
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
  for (int d = D + tid; d < DP; d += kDecThreads) sq[d] = 0.f;
  __syncthreads();

  const int r1 = min(S, r0 + rps);  // valid rows of this split: [r0, r1)
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

  auto consume = [&](int cur, auto u) {
    constexpr int U = decltype(u)::value;
    float dot2[2] = {0.f, 0.f};  // two independent chains
#pragma unroll
    for (int k = 0; k < MAXC; ++k) {
      const T* e = reinterpret_cast<const T*>(&kr[U][k]);
#pragma unroll
      for (int j = 0; j < EPC; ++j) dot2[j & 1] = fmaf(E::to_f(e[j]), qv[k][j], dot2[j & 1]);
    }
    float dot = dot2[0] + dot2[1];
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
        const T* e = reinterpret_cast<const T*>(&vr[U][k]);
#pragma unroll
        for (int j = 0; j < EPC; ++j) z[k][j] = fmaf(pr, E::to_f(e[j]), z[k][j]);
      }
    }
  };
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;
  using I3 = std::integral_constant<int, 3>;
  constexpr int RS = 16 * kDecWaves;  // rows per step of the workgroup
  for (int row = row0; row - wave * 16 - rr < r1; row += 4 * RS) {
    fetch(row + 3 * RS, I3{});
    consume(row, I0{});
    fetch(row + 4 * RS, I0{});
    consume(row + RS, I1{});
    fetch(row + 5 * RS, I1{});
    consume(row + 2 * RS, I2{});
    fetch(row + 6 * RS, I2{});
    consume(row + 3 * RS, I3{});
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
  // merge the waves -> this split's partial
  {
    float mw[kDecWaves];
    float M = kNegInf;
#pragma unroll
    for (int w = 0; w < kDecWaves; ++w) {
      mw[w] = red[w * (DP + 2)];
      M = fmaxf(M, mw[w]);
    }
    const float Ms = M == kNegInf ? 0.f : M;
    float* part = p.part + (int64_t(bh) * p.nsplit + split) * (D + 2);
    for (int d = tid; d < D; d += kDecThreads) {
      float zs = 0.f;
#pragma unroll
      for (int w = 0; w < kDecWaves; ++w) zs += red[w * (DP + 2) + 2 + d] * fexp2(mw[w] - Ms);
      store_coherent(part + 2 + d, zs);
    }
    if (tid == 0) {
      float L = 0.f;
#pragma unroll
      for (int w = 0; w < kDecWaves; ++w) L += red[w * (DP + 2) + 1] * fexp2(mw[w] - Ms);
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

// Splits per head: about three workgroups per CU over the whole batch (a multiple of the CU count,
// so no CU runs one more than the others), but no split shorter than 512 rows at full capacity
// (every split costs a published partial, a completion count and a share of the merge).
static int device_cus() {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      cus <= 0)
    return 256;
  return cus;
}
static int decode_splits(const mote_relation_decode_args* a) {
  const int64_t BH = int64_t(a->B) * a->H;
  int64_t n = (3 * int64_t(device_cus()) + BH - 1) / BH;
  const int64_t by_rows = (int64_t(a->capacity) + 511) / 512;
  if (n > by_rows) n = by_rows;
  if (n > kDecMaxSplits) n = kDecMaxSplits;
  return int(n < 1 ? 1 : n);
}

struct DecWs {
  size_t part, cnt, cnt_seq, total;
};
static DecWs decode_ws(const mote_relation_decode_args* a) {
  const int nsplit = decode_splits(a);
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
  p.nsplit = decode_splits(a);
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
    hipLaunchKernelGGL((relation_decode_kernel<T_, DP_>), dim3(grid), dim3(kDecThreads), shmem, stream, p);          \
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
