// One decode step of one Relation layer (mote/infer/graph.py:151-187), one launch.
//
// Grid: nsplit x (B*H) workgroups, block id = split * (B*H) + head index; nsplit is a host choice
// from the shape only, so the launch can be captured in a HIP graph. Each head's cache is read in
// steps of 64 rows (4 waves, 16 rows per wave, 4 lanes per row, 16-byte loads of P2 and I~), and
// the steps are dealt to the splits round-robin: split s takes steps s, s + nsplit, s + 2 nsplit, ...
// Two things follow. The addresses of a split's first steps do not depend on the position S, so
// the first three steps of loads are issued at the very start, while S and the new row are still
// in flight; and for every S the splits' step counts differ by at most one. A ring of four register
// sets keeps three steps of loads in flight while one step computes U_j = <q, P2_j> / sqrt(D),
// e_j = SiLU(U_j) in log2 units and an online softmax per row group (running max raised lazily, by
// more than 2^8 only).
//
// Merge within the workgroup through LDS: the workgroup's largest running max M, every row group
// rescaled to it, the 64 row groups' z written as rows of an LDS table and summed per column in a
// fixed order. The split publishes (M, l, z[D]) with agent-coherent stores, waits for their
// completion, then counts itself with one atomic add on its head's counter (each counter on a
// cache line of its own: counters that share a line serialise every split of every head). Every
// split counts, rows or not, so the count never depends on S. The workgroup that brings the count
// to nsplit reads all partials back with agent-coherent loads (one batch) and finishes the head:
// merge in a fixed order, the Self score from the new row, g = sigmoid(LSE - lam ln(S+1) - S_self),
// Y = (1-g) I~_S + g z/l, the append of the new P2 / I~ row at S and the reset of the counter. With
// MOTE_DECODE_ADVANCE or an xm output, a second counter per sequence picks the last head to finish:
// it adds 1 to S[b] (by then every workgroup of the sequence has read S[b]) and writes xm. Counters start at zero (the workspace is zeroed once) and every call
// leaves them zero.
//
// The new rows (graph.py:158-172) are computed by every workgroup in its prologue, under the
// latency of the first loads: the query and the new P2 row RoPE'd at S, I~ Givens-rotated with its
// partner head's raw row, all rounded to the cache dtype. Bandwidth-bound by design: no MFMA.
#include <mutex>
#include <type_traits>

#include "common.hpp"
#include "params.hpp"

namespace mote {

struct DecParams {
  const float* lam;
  const float* inv_freq;  // never null: without RoPE / Givens the launcher points both at lam
  const float* theta;
  int rope, givens;       // whether inv_freq / theta are the real tables
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
  float* xm;          // [B] mean over heads of g, or null
  const unsigned char* run;  // predicate: 0 -> the launch writes nothing (null: always run)
  float* part;        // [BH][nsplit][D + 2]  (max, l, z)
  int* cnt;           // [BH] splits published in this call, kDecCntStride ints apart (zero between calls)
  int* cnt_seq;       // [B] heads finished in this call, kDecCntStride ints apart (zero between calls)
  int B, H, D, cap, parity, flags, nsplit;
  float scale, tau_inv;
};

constexpr int kDecMaxSplits = 64;   // the merge gives every split one lane of a wave
constexpr int kDecWaves = 4;        // waves per workgroup
constexpr int kDecThreads = 64 * kDecWaves;
constexpr int kDecRows = 16 * kDecWaves;  // rows of one step
constexpr int kDecCntStride = 64;   // ints between two completion counters: 256 bytes

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

template <typename T, int DP>
__global__ void __launch_bounds__(kDecThreads)
relation_decode_kernel(const DecParams p) {
  using E = Elem<T>;
  constexpr int EPC = 16 / sizeof(T);
  constexpr int MAXC = (DP / EPC + 3) / 4;  // 16-byte chunks per lane (lane c owns chunks c, c+4, ...)
  constexpr int ZS = DP + 4;                // LDS row of one row group's z (16-byte aligned)
  __shared__ __align__(16) float zred[kDecRows * ZS];  // row-group z, then the head's partials
  __shared__ float sq[DP], knew[DP], inew[DP];
  __shared__ float csum[2][DP];
  __shared__ float sm[kDecWaves], sl[kDecWaves];
  __shared__ float wsp[kDecMaxSplits];
  __shared__ float sML[3];
  __shared__ int s_last;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int BH = p.B * p.H;
  const int bh = blockIdx.x % BH;
  const int split = blockIdx.x / BH;
  const int b = bh / p.H, h = bh % p.H;
  const int D = p.D, half = D / 2;
  const int nch = D / EPC;
  const int nsp = p.nsplit;
  const int rr = lane >> 2, c = lane & 3;
  const int roff = wave * 16 + rr;  // this lane's row within a step
  const T* kbase = reinterpret_cast<const T*>(p.kc) + b * p.kc_sb + h * p.kc_sh;
  const T* vbase = reinterpret_cast<const T*>(p.vc) + b * p.vc_sb + h * p.vc_sh;

  // The small loads go first and unconditionally (lanes past the row read a clamped element):
  // loads complete in order, so the new rows can be computed while the cache loads issued after
  // them are still in flight. Wave 0 takes the query and P2 halves, waves 2-3 the I~ row and its
  // Givens partner: pairing by layer parity (relation.py:150-174), even layers (0,1),(2,3)...,
  // odd layers (1,2),...,(H-1,0); the first head of a pair gets c a - s b, the second s a + c b.
  // lam and theta are read per lane through an index the compiler cannot see is zero: as scalar
  // loads they would be waited for at the first barrier (whose wait for the LDS writes also waits
  // for every scalar load in flight).
  int vzero;
  asm volatile("v_mov_b32 %0, 0" : "=v"(vzero));
  const float lam = p.lam[vzero];
  // S and the predicate byte also go before the cache loads (whose addresses do not depend on
  // them): the new rows and the predicate's test then wait for none of the cache loads. Without a
  // predicate any valid byte is read.
  const int64_t S64 = p.S[b + vzero];
  const int run_v = (p.run ? p.run : reinterpret_cast<const unsigned char*>(p.lam))[vzero];
  // Written as integer arithmetic: the compiler turns selects here into branches, and a branch
  // would split the kernel-argument loads over two waits.
  const int odd = h & 1, par = p.parity;
  const bool first = (odd ^ par) == 0;
  int nb = h + 2 * odd - 1;  // odd layers: h + 1 for odd h, h - 1 for even h, modulo H
  nb += int(nb < 0) * p.H - int(nb >= p.H) * p.H;
  const int other = (h ^ 1) + par * (nb - (h ^ 1));
  const int pair = (h >> 1) + (par & (odd ^ 1)) * ((other >> 1) - (h >> 1));
  const float th = p.theta[(p.givens ? pair : 0) + vzero];
  const int qi = min(tid, half - 1);
  const int di = min(tid & 127, D - 1);
  const T* in_b = reinterpret_cast<const T*>(p.p1) + b * p.in_sb + h * D;
  const float q0 = E::to_f(in_b[qi]), q1 = E::to_f(in_b[qi + half]);
  const T* kn_b = reinterpret_cast<const T*>(p.p2) + b * p.in_sb + h * D;
  const float k0 = E::to_f(kn_b[qi]), k1 = E::to_f(kn_b[qi + half]);
  const T* i_raw = reinterpret_cast<const T*>(p.info) + b * p.in_sb;
  const float iself = E::to_f(i_raw[h * D + di]), ioth = E::to_f(i_raw[other * D + di]);
  const float invf = p.inv_freq[p.rope ? qi : 0];

  // A ring of four register sets, one step each, named by constants (a copy between sets would
  // make the compiler wait for the newest loads before issuing the next ones). Loads are
  // unconditional: rows are clamped to rlim (the cache's last row until S is known, then the
  // split's last valid row, so loads past the split re-read lines already fetched), and chunks
  // past the head dim to its last chunk; the math ignores both. A load under a lane condition would
  // hide from the compiler's count of outstanding loads, and it would then wait for all of them.
  Chunk kr[4][MAXC], vr[4][MAXC];
  int rlim = p.cap - 1;
  auto fetch = [&](int j, auto u) {
    constexpr int U = decltype(u)::value;
    const int rc = min((split + j * nsp) * kDecRows + roff, rlim);
#pragma unroll
    for (int k = 0; k < MAXC; ++k) {
      const int kc = min(c + 4 * k, nch - 1);
      kr[U][k] = load_chunk(kbase + int64_t(rc) * p.kc_sr + kc * EPC);
      vr[U][k] = load_chunk(vbase + int64_t(rc) * p.vc_sr + kc * EPC);
    }
  };
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;
  using I3 = std::integral_constant<int, 3>;
  fetch(0, I0{});
  fetch(1, I1{});
  fetch(2, I2{});
  asm volatile("" ::: "memory");  // keeps the predicate's test (an early exit) after the cache loads

  // The predicate (a device flag, e.g. the router's boundary bit): with 0 every workgroup leaves
  // here, before any write, count or barrier, so a captured step costs one empty launch when the
  // chunk is not a boundary (graph.py:224-226 skips the step with a conditional node instead).
  if (p.run && run_v == 0) return;
  const bool bad = S64 < 0 || S64 >= p.cap;
  const int S = bad ? 0 : int(S64);

  // the new rows at S, computed on every lane (a use under a lane condition would let the compiler
  // sink the small loads behind the cache loads); only the owning lanes write them to LDS
  float cs, sn;
  sincosf((float)S * invf, &sn, &cs);
  // MOTE_DECODE_ROPE_F32: fp32 tables and fp32 arithmetic, one rounding at the end (the rows are
  // computed both ways and selected, so the flag adds no branch ahead of the cache loads)
  const bool rope32 = (p.flags & MOTE_DECODE_ROPE_F32) != 0;
  const float cs32 = p.rope ? cs : 1.f, sn32 = p.rope ? sn : 0.f;
  cs = p.rope ? round_to<T>(cs) : 1.f;
  sn = p.rope ? round_to<T>(sn) : 0.f;
  const float rq0 = rope32 ? round_to<T>(rot_round<float>(q0, cs32, q1, -sn32)) : rot_round<T>(q0, cs, q1, -sn);
  const float rq1 = rope32 ? round_to<T>(rot_round<float>(q1, cs32, q0, sn32)) : rot_round<T>(q1, cs, q0, sn);
  const float rk0 = rope32 ? round_to<T>(rot_round<float>(k0, cs32, k1, -sn32)) : rot_round<T>(k0, cs, k1, -sn);
  const float rk1 = rope32 ? round_to<T>(rot_round<float>(k1, cs32, k0, sn32)) : rot_round<T>(k1, cs, k0, sn);
  float gc, gs;
  sincosf(th, &gs, &gc);
  gc = p.givens ? round_to<T>(gc) : 1.f;
  gs = p.givens ? round_to<T>(gs) : 0.f;
  const float rin = p.givens ? rot_round<T>(iself, gc, ioth, first ? -gs : gs) : iself;
  if (tid < half) {
    sq[tid] = rq0;
    sq[tid + half] = rq1;
    knew[tid] = rk0;
    knew[tid + half] = rk1;
  } else if (tid >= 128 && tid < 128 + D) {
    inew[tid - 128] = rin;
  }
  for (int d = D + tid; d < DP; d += kDecThreads) sq[d] = 0.f;
  __syncthreads();

  // this split's steps: s + j nsplit for j < ns, rows below S
  const int nst = (S + kDecRows - 1) / kDecRows;
  const int ns = nst > split ? (nst - split + nsp - 1) / nsp : 0;
  rlim = ns > 0 ? min((split + (ns - 1) * nsp) * kDecRows + kDecRows, S) - 1 : 0;

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

  const float c2 = p.scale * kLog2e;
  // Steps past the split are skipped whole (ns is uniform): their loads, clamped to lines already
  // fetched, are never waited for.
  auto consume = [&](int jstep, auto u) {
    constexpr int U = decltype(u)::value;
    if (jstep >= ns) return;
    float dot2[2] = {0.f, 0.f};  // two independent chains
#pragma unroll
    for (int k = 0; k < MAXC; ++k) {
      const T* e = reinterpret_cast<const T*>(&kr[U][k]);
#pragma unroll
      for (int j = 0; j < EPC; ++j) dot2[j & 1] = fmaf(E::to_f(e[j]), qv[k][j], dot2[j & 1]);
    }
    float dot = dot2[0] + dot2[1];
    dot += dpp<kDppXor1>(dot);  // the row's four lanes: the sum of xor 1 then xor 2 in every lane
    dot += dpp<kDppXor2>(dot);
    const int row = (split + jstep * nsp) * kDecRows + roff;
    if (row < S) {
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
  for (int j = 0; j < ns; j += 4) {
    fetch(j + 3, I3{});
    consume(j, I0{});
    fetch(j + 4, I0{});
    consume(j + 1, I1{});
    fetch(j + 5, I1{});
    consume(j + 2, I2{});
    fetch(j + 6, I2{});
    consume(j + 3, I3{});
  }

  // ---- merge of the 64 row groups (lanes of one row group hold the same m and l) ----
  // over the wave's 16 row groups (lanes with equal lane & 3), in lane 0 the xor butterfly 4, 8, 16,
  // 32: lane + 4 and lane ^ 8 within the row give lane 0 the partners xor 4 / 8 would, then the row
  // swaps
  float mw = fmaxf(m, dpp<kDppNext4>(m));
  mw = lanegroup_max(fmaxf(mw, dpp<kDppRor8>(mw)));
  if (lane == 0) sm[wave] = mw;
  __syncthreads();
  float M = sm[0];
#pragma unroll
  for (int w = 1; w < kDecWaves; ++w) M = fmaxf(M, sm[w]);
  const float a = fexp2(m - (M == kNegInf ? 0.f : M));  // 0 for a row group without rows
  float lw = l * a;
  lw += dpp<kDppNext4>(lw);
  lw = lanegroup_sum(lw + dpp<kDppRor8>(lw));
  if (lane == 0) sl[wave] = lw;
  float* zg = zred + roff * ZS;
#pragma unroll
  for (int k = 0; k < MAXC; ++k) {
    const int kc = c + 4 * k;
    if (kc < nch)
#pragma unroll
      for (int j = 0; j < EPC; ++j) zg[kc * EPC + j] = z[k][j] * a;
  }
  __syncthreads();
  {
    const int d = tid & 127, hf = tid >> 7;  // two halves of 32 row groups per column
    if (d < D) {
      const float* col = zred + hf * 32 * ZS + d;
      float s0 = 0.f, s1 = 0.f;
#pragma unroll
      for (int g2 = 0; g2 < 32; g2 += 2) {
        s0 += col[g2 * ZS];
        s1 += col[(g2 + 1) * ZS];
      }
      csum[hf][d] = s0 + s1;
    }
  }
  __syncthreads();
  {
    float* part = p.part + (int64_t(bh) * nsp + split) * (D + 2);
    if (tid < D) store_coherent(part + 2 + tid, csum[0][tid] + csum[1][tid]);
    if (tid == 0) {
      float L = 0.f;
#pragma unroll
      for (int w = 0; w < kDecWaves; ++w) L += sl[w];
      store_coherent(part, M);
      store_coherent(part + 1, L);
    }
  }
  // Publish, then count. The ordering comes from the gfx942-family memory model (LLVM AMDGPUUsage,
  // "Memory Model GFX942", which gfx950 follows), not from a release / acquire pair: monotonic
  // atomic stores and loads at agent scope are issued with sc1 (read off the ISA: global_store /
  // global_load ... sc1), so the stores write through the XCD's L2 to the device-coherent level and
  // the loads do not hit a stale L2 line; s_waitcnt vmcnt(0) returns once every store of the wave is
  // acknowledged there. After the barrier all partials of the workgroup are visible device-wide,
  // before the count's atomic add is even issued; the workgroup that sees the last count reads them
  // with agent-scope atomic loads after its add has returned. A release add / acquire load would add
  // an L2 writeback and invalidate per workgroup (buffer_wbl2 sc1 / buffer_inv sc1) for data that
  // never sits in L2.
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (tid == 0) {
    const int before = __hip_atomic_fetch_add(p.cnt + bh * kDecCntStride, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = before == nsp - 1;
  }
  __syncthreads();
  if (!s_last) return;

  // ---- the last workgroup of the head: all partials in one batch of loads ----
  const int np = nsp * (D + 2);
  const float* pb = p.part + int64_t(bh) * np;
  constexpr int KP = (kDecMaxSplits * (DP + 2) + kDecThreads - 1) / kDecThreads;
  float pv[KP];
#pragma unroll
  for (int k = 0; k < KP; ++k) pv[k] = load_coherent(pb + min(tid + k * kDecThreads, np - 1));
#pragma unroll
  for (int k = 0; k < KP; ++k)
    if (tid + k * kDecThreads < np) zred[tid + k * kDecThreads] = pv[k];
  __syncthreads();
  const int stride = D + 2;
  if (wave == 0) {
    // split weights 2^(m_s - Mh) and L = sum_s l_s 2^(m_s - Mh), one split per lane
    const float ms = lane < nsp ? zred[lane * stride] : kNegInf;
    const float mx = wave_max(ms);
    const float Mh = mx == kNegInf ? 0.f : mx;
    const float w = fexp2(ms - Mh);
    if (lane < nsp) wsp[lane] = w;
    const float ls = wave_sum_lane0(lane < nsp ? zred[lane * stride + 1] * w : 0.f);
    if (lane == 0) {
      sML[0] = Mh;
      sML[1] = ls;
    }
  } else if (wave == 1) {
    // Self score U_SS = <q, P2_S> / sqrt(D)
    float u = 0.f;
    for (int d = lane; d < D; d += 64) u = fmaf(sq[d], knew[d], u);
    u = wave_sum_lane0(u);
    if (lane == 0) sML[2] = u;
  }
  __syncthreads();
  const float Mh = sML[0], L = sML[1];
  const float sself = sigmoid_acc(sML[2] * p.scale * p.tau_inv);
  const bool has = L > 0.f;
  const float lse = has ? (Mh + __log2f(L)) * kLn2 : kNegInf;
  const float gate = has ? sigmoid_acc(lse - lam * logf((float)S + 1.0f) - sself) : 0.f;
  const float invL = has ? 1.0f / L : 0.f;
  T* y = reinterpret_cast<T*>(p.y) + b * p.y_sb + h * D;
  T* kw = reinterpret_cast<T*>(p.kc) + b * p.kc_sb + h * p.kc_sh + int64_t(S) * p.kc_sr;
  T* vw = reinterpret_cast<T*>(p.vc) + b * p.vc_sb + h * p.vc_sh + int64_t(S) * p.vc_sr;
  for (int d = tid; d < D; d += kDecThreads) {
    float zsum = 0.f;
#pragma unroll 8
    for (int s2 = 0; s2 < nsp; ++s2) zsum = fmaf(zred[s2 * stride + 2 + d], wsp[s2], zsum);
    const float yv = (1.0f - gate) * inew[d] + gate * zsum * invL;
    y[d] = E::from_f(bad ? __builtin_nanf("") : yv);
    if (!bad) {
      kw[d] = E::from_f(knew[d]);
      vw[d] = E::from_f(inew[d]);
    }
  }
  if (tid == 0) {
    const float gv = bad ? __builtin_nanf("") : gate;
    __hip_atomic_store(p.cnt + bh * kDecCntStride, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    // The per-sequence count only serves the advance of S and xm; without either there is nothing
    // to count, and the last workgroup ends without waiting for an atomic's return.
    p.g[bh] = gv;
    if ((p.flags & MOTE_DECODE_ADVANCE) || p.xm) {
      // the last head of the sequence: every workgroup of the sequence has read S[b] by now. With xm
      // the count is acquire-release, so the last head also sees every other head's g (measured
      // against g published with coherent stores and a relaxed count: 1 % slower per engine token).
      int before;
      if (p.xm)
        before = __hip_atomic_fetch_add(p.cnt_seq + b * kDecCntStride, 1, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
      else
        before = __hip_atomic_fetch_add(p.cnt_seq + b * kDecCntStride, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (before == p.H - 1) {
        __hip_atomic_store(p.cnt_seq + b * kDecCntStride, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (p.flags & MOTE_DECODE_ADVANCE) p.S[b] = S64 + 1;
        if (p.xm) {
          float sum = 0.f;  // fixed head order
          for (int hh = 0; hh < p.H; ++hh) sum += p.g[b * p.H + hh];
          p.xm[b] = sum / float(p.H);
        }
      }
    }
  }
}

// Splits per head: one workgroup per CU over the whole batch (measured at Mote-96M, batch 1 and
// 16: more splits add completion counts and merge work without speeding up the sweep, fewer leave
// CUs idle), at least two steps per split at full capacity, and at most one split per lane of the
// merging wave.
static int device_cus() {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      cus <= 0)
    return 256;
  return cus;
}
static int decode_splits(const mote_relation_decode_args* a) {
  const int64_t BH = int64_t(a->B) * a->H;
  int64_t n = int64_t(device_cus()) / BH;
  const int64_t by_rows = (int64_t(a->capacity) + 2 * kDecRows - 1) / (2 * kDecRows);
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
  const size_t line = kDecCntStride * sizeof(int);
  DecWs w;
  w.part = 0;
  w.cnt = (BH * size_t(nsplit) * size_t(a->D + 2) * sizeof(float) + line - 1) / line * line;
  w.cnt_seq = w.cnt + BH * line;
  w.total = w.cnt_seq + size_t(a->B) * line;
  return w;
}

size_t decode_workspace_bytes(const mote_relation_decode_args* a) { return decode_ws(a).total; }

static int check_decode_args(const mote_relation_decode_args* a, const char* what) {
  if (!a) return set_error(MOTE_ERR_ARGUMENT, "%s: null args", what);
  if (a->dtype != MOTE_F32 && a->dtype != MOTE_BF16) return set_error(MOTE_ERR_ARGUMENT, "%s: bad dtype %d", what, a->dtype);
  if (a->D <= 0 || a->D > 128 || a->D % 8 != 0)
    return set_error(MOTE_ERR_SHAPE, "%s: head dim %d unsupported (need 8 <= D <= 128, D %% 8 == 0)", what, a->D);
  if (a->B <= 0 || a->H <= 0 || a->H % 2 || a->capacity <= 0) return set_error(MOTE_ERR_SHAPE, "%s: bad sizes", what);
  if (!a->lam || !a->S || !a->p1 || !a->p2 || !a->info || !a->cache_p2.data || !a->cache_info.data || !a->y || !a->g)
    return set_error(MOTE_ERR_ARGUMENT, "%s: null pointer", what);
  return MOTE_OK;
}

// The launch itself, with the partials and counters at base + the offsets of `w`.
static int launch_decode_ws(const mote_relation_decode_args* a, void* ws_base, const DecWs& w, hipStream_t stream) {
  DecParams p;
  p.lam = a->lam; p.S = a->S;
  p.rope = a->inv_freq != nullptr;
  p.givens = a->theta != nullptr;
  p.inv_freq = p.rope ? a->inv_freq : a->lam;
  p.theta = p.givens ? a->theta : a->lam;
  p.p1 = a->p1; p.p2 = a->p2; p.info = a->info; p.in_sb = a->in_sb;
  p.kc = a->cache_p2.data; p.kc_sb = a->cache_p2.stride_b; p.kc_sh = a->cache_p2.stride_h; p.kc_sr = a->cache_p2.stride_r;
  p.vc = a->cache_info.data; p.vc_sb = a->cache_info.stride_b; p.vc_sh = a->cache_info.stride_h; p.vc_sr = a->cache_info.stride_r;
  p.y = a->y; p.y_sb = a->y_sb; p.g = a->g;
  const size_t BH = size_t(a->B) * a->H;
  p.nsplit = decode_splits(a);
  char* ws = reinterpret_cast<char*>(ws_base);
  p.part = reinterpret_cast<float*>(ws + w.part);
  p.cnt = reinterpret_cast<int*>(ws + w.cnt);
  p.cnt_seq = reinterpret_cast<int*>(ws + w.cnt_seq);
  p.xm = a->xm;
  p.run = a->run;
  p.B = a->B; p.H = a->H; p.D = a->D; p.cap = a->capacity; p.parity = a->layer_parity & 1; p.flags = a->flags;
  p.scale = 1.0f / sqrtf((float)a->D);
  p.tau_inv = 1.0f / a->tau_s;
  const int grid = int(BH) * p.nsplit;
  const int DP = padded_dim(a->D);
#define MOTE_DEC_LAUNCH(T_, DP_)                                                                               \
  do {                                                                                                       \
    hipLaunchKernelGGL((relation_decode_kernel<T_, DP_>), dim3(grid), dim3(kDecThreads), 0, stream, p);          \
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

int launch_decode(const mote_relation_decode_args* a, hipStream_t stream) {
  if (const int rc = check_decode_args(a, "relation_decode")) return rc;
  if (!a->workspace || a->workspace_bytes < decode_workspace_bytes(a))
    return set_error(MOTE_ERR_WORKSPACE, "relation_decode: workspace of %zu bytes, %zu needed", a->workspace_bytes,
                     decode_workspace_bytes(a));
  return launch_decode_ws(a, a->workspace, decode_ws(a), stream);
}

// ------------------------------------------------------------------------------------------------
// The no-allocation entry point: the partials and counters live in `scratch`, a static device array
// (one copy per GPU, alive until the process ends) of MOTE_DECODE_STATIC_SLOTS slots; a call uses the
// slot its `static_slot` names, so calls on different slots never touch the same bytes. In host code
// `scratch` names a host-side stand-in, not device memory: its device address comes from
// hipGetSymbolAddress, once per device (with that device current), and only that address (plus a
// slot offset) is ever handed to a kernel. The first call on a slot of a device clears that slot with
// a fill kernel in the caller's stream order. Calls on one slot of one GPU share it.
//
// Layout. The completion counters must be zero when a call starts. A call leaves the counters it
// used at zero, but the workspace layout (counters after the partials) moves them with the shape, so
// in a shared array a smaller call's counters would land on a larger call's stale partials. Here the
// counters have fixed slots at the front instead: sequence counter b in line b, head counter bh in
// line kStaticSeqLines + bh, 256 bytes each; every slot is either untouched since the clear or
// reset by its last user. The partials follow; their contents never need to start at zero.
// ------------------------------------------------------------------------------------------------
constexpr int kStaticSeqLines = 256;    // sequences per call
constexpr int kStaticHeadLines = 1024;  // sequence-heads per call
static DecWs decode_ws_static(const mote_relation_decode_args* a) {
  const size_t line = kDecCntStride * sizeof(int);
  DecWs w;
  w.cnt_seq = 0;
  w.cnt = size_t(kStaticSeqLines) * line;
  w.part = w.cnt + size_t(kStaticHeadLines) * line;
  w.total = w.part + size_t(a->B) * a->H * size_t(decode_splits(a)) * size_t(a->D + 2) * sizeof(float);
  return w;
}

static __device__ __align__(256) unsigned char scratch[size_t(MOTE_DECODE_STATIC_SLOTS) * MOTE_DECODE_STATIC_BYTES];

constexpr int kMaxScratchDevices = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[kMaxScratchDevices];  // device address of `scratch` per device, once known
static bool g_slot_clear[kMaxScratchDevices][MOTE_DECODE_STATIC_SLOTS];  // slot cleared on that device

__global__ void __launch_bounds__(256) clear_scratch_kernel(uint4* p, int n16) {
  for (int i = blockIdx.x * 256 + threadIdx.x; i < n16; i += gridDim.x * 256) p[i] = make_uint4(0u, 0u, 0u, 0u);
}

static int scratch_address(hipStream_t stream, int slot, void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxScratchDevices)
    return set_error(MOTE_ERR_LAUNCH, "relation_decode_static: no usable current device");
  if (stream) {
    int sdev = -1;
    if (hipStreamGetDevice(stream, &sdev) != hipSuccess || sdev != dev)
      return set_error(MOTE_ERR_ARGUMENT, "relation_decode_static: the stream's device (%d) must be the current one (%d)",
                       sdev, dev);
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_slot_clear[dev][slot]) {
    // the clear must run once, not on every replay of a graph: refuse a first call under capture
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if (stream && hipStreamIsCapturing(stream, &cap) == hipSuccess && cap != hipStreamCaptureStatusNone)
      return set_error(MOTE_ERR_ARGUMENT, "relation_decode_static: the first call on slot %d of a device clears that "
                                          "slot and must not be captured; call it once outside the capture first", slot);
    if (!g_scratch_ptr[dev]) {
      void* ptr = nullptr;
      const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
      if (e != hipSuccess || !ptr)
        return set_error(MOTE_ERR_LAUNCH, "relation_decode_static: hipGetSymbolAddress failed: %s", hipGetErrorString(e));
      g_scratch_ptr[dev] = ptr;
    }
    unsigned char* base = static_cast<unsigned char*>(g_scratch_ptr[dev]) + size_t(slot) * MOTE_DECODE_STATIC_BYTES;
    hipLaunchKernelGGL(clear_scratch_kernel, dim3(64), dim3(256), 0, stream, reinterpret_cast<uint4*>(base),
                       int(MOTE_DECODE_STATIC_BYTES / 16));
    if (const int rc = check_launch("relation_decode_static (scratch clear)")) return rc;
    g_slot_clear[dev][slot] = true;
  }
  *out = static_cast<unsigned char*>(g_scratch_ptr[dev]) + size_t(slot) * MOTE_DECODE_STATIC_BYTES;
  return MOTE_OK;
}

int launch_decode_static(const mote_relation_decode_args* a, hipStream_t stream) {
  if (const int rc = check_decode_args(a, "relation_decode_static")) return rc;
  const DecWs w = decode_ws_static(a);
  if (a->B > kStaticSeqLines || int64_t(a->B) * a->H > kStaticHeadLines || w.total > MOTE_DECODE_STATIC_BYTES)
    return set_error(MOTE_ERR_WORKSPACE,
                     "relation_decode_static: B = %d sequences x H = %d heads need %zu bytes of scratch with at most "
                     "%d sequences and %d sequence-heads; a slot of the static array holds %u (use mote_relation_decode with a "
                     "workspace)", a->B, a->H, w.total, kStaticSeqLines, kStaticHeadLines,
                     unsigned(MOTE_DECODE_STATIC_BYTES));
  if (a->static_slot < 0 || a->static_slot >= MOTE_DECODE_STATIC_SLOTS)
    return set_error(MOTE_ERR_ARGUMENT, "relation_decode_static: static_slot = %d, want 0 to %d", a->static_slot,
                     MOTE_DECODE_STATIC_SLOTS - 1);
  void* ws = nullptr;
  if (const int rc = scratch_address(stream, a->static_slot, &ws)) return rc;
  return launch_decode_ws(a, ws, w, stream);
}

}  // namespace mote
