// Fused Relation backward for gfx950 (mote/model/flash_relation.py:10-15 for the algebra).
//
// Three stages, all on the caller's stream:
//
// 1. rows (one workgroup per 64 query rows of one (batch, head)): the per-row terms
//      dI-bar = g dY, dg = dY.(I-bar - I~_i), dA = dg g (1-g), Delta = dI-bar.I-bar,
//      dU_ii = -dA S (1-S) / tau, dlam partial = -sum dA ln(i+1)
//    and the operand copies the main kernels stage from: Q and dI-bar padded to the kernel's head
//    dim, row-major and transposed (head-dim major), c = dA - Delta, lse in log2 units (+inf for
//    padding rows and rows without a past, which zeroes their weights), and the fp32 dP1
//    accumulator initialised with the Self part dU_ii P2_i / sqrt(D).
// 2. key blocks (one workgroup per 64 keys of one (batch, head), 4 waves x 16 keys, longest
//    first): walks every query block that can see its keys and per block computes
//      U = Q K^T and dW = dI-bar V^T (keys in the accumulator columns, so the results feed the
//      next products as permuted-k A operands without a transpose),
//      w = exp(SiLU(U) - L), dE = w (dW - Delta + dA), dU = dE SiLU'(U),
//      dV += W^T dI-bar, dK += dU^T Q (registers, all query blocks),
//      and, in the one-pass mode, dQ = dU K over the 64 keys (dU through LDS) added to the fp32
//      accumulator with hardware float atomics.
//    The Self terms of key rows that are also queries, (1-g) dY into dI~ and dU_ii P1 into dP2,
//    are added before the single store.
// 3. one-pass: dP1 accumulator -> output dtype. Deterministic mode: a query-stationary kernel
//    recomputes w and dU per (query block, key block) and accumulates dQ in registers instead of
//    atomics (the reference's two-pass `_bwd_q_kernel`, flash_relation.py:419-460), so every
//    result is bitwise reproducible. dlam: a fixed-order sum of the row partials.
#include "common.hpp"
#include "bwd.hpp"

namespace mote {


// ------------------------------------------------------------------------------------------------
// 1. rows
// ------------------------------------------------------------------------------------------------
// LEAN (tile kernels): only dI-bar rows, the per-block stats, dU_ii and the dlam partials; the
// register-staged kernels also need the P1 copies, both transposes and the dP1 accumulator.
template <typename T, int DP, bool LEAN>
__global__ void __launch_bounds__(256) bwd_rows_kernel(const BwdParams p) {
  using E = Elem<T>;
  constexpr int EPC = 16 / sizeof(T);       // elements per 16-byte chunk
  constexpr int CPR = DP / EPC;             // chunks per row
  constexpr int NCH = kRowBlock * CPR;      // chunks per block
  constexpr int CT = (NCH + 255) / 256;     // chunks per thread
  constexpr int LD = DP + EPC;              // LDS row stride (elements)
  __shared__ __align__(16) T sq[LEAN ? 1 : kRowBlock * LD];
  __shared__ __align__(16) T sd[LEAN ? 1 : kRowBlock * LD];
  __shared__ float part[3][kRowBlock][CPR + 1];
  __shared__ float sdu[kRowBlock];
  __shared__ float sred[kRowBlock];

  const int bh = blockIdx.y;
  const int b = bh / p.H, h = bh % p.H;
  const int i0 = blockIdx.x * kRowBlock;
  const int tid = threadIdx.x;
  const int D = p.D;
  const T* qb = reinterpret_cast<const T*>(p.p1) + b * p.q_sb + h * p.q_sh;
  const T* kb = reinterpret_cast<const T*>(p.p2) + b * p.k_sb + h * p.k_sh;
  const T* vb = reinterpret_cast<const T*>(p.info) + b * p.v_sb + h * p.v_sh;
  const T* yb = reinterpret_cast<const T*>(p.dy) + b * p.y_sb + h * p.y_sh;
  T* wq = LEAN ? nullptr : reinterpret_cast<T*>(p.wq) + (int64_t(bh) * p.TQp + i0) * DP;
  T* wd = reinterpret_cast<T*>(p.wdib) + (int64_t(bh) * p.TQp + i0) * DP;
  // the fused key + query launch's control words: this block's count, and block (0, 0) the job
  // counters (agent-scope stores, as that launch reads and adds them)
  if (LEAN && p.kvq && tid == 0) {
    const int nqb = p.TQp / kRowBlock;
    __hip_atomic_store(p.kvq + kKvqCounts + bh * nqb + blockIdx.x, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (blockIdx.x == 0 && bh == 0) {
      for (int q = 0; q < 8; ++q)
        __hip_atomic_store(p.kvq + kKvqJob + q * kKvqJobStride, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }

  // pass 1: 16-byte chunks; per-chunk partial dot products, dI-bar and the row-major copies
  Chunk kreg[CT];
#pragma unroll
  for (int c = 0; c < CT; ++c) {
    const int idx = tid + 256 * c;
    if (idx >= NCH) break;
    const int r = idx / CPR, cc = idx % CPR;
    const int i = i0 + r;
    const int d0 = cc * EPC;
    const bool ok = i < p.TQ && d0 < D;
    const int qa = p.q_start + i;
    Chunk cq = zero_chunk(), ck = zero_chunk(), cv = zero_chunk(), cy = zero_chunk();
    float ibv[EPC];
    float gi = 0.f;
    if (ok) {
      cq = load_chunk(qb + int64_t(i) * p.q_sr + d0);
      ck = load_chunk(kb + int64_t(qa) * p.k_sr + d0);
      cv = load_chunk(vb + int64_t(qa) * p.v_sr + d0);
      cy = load_chunk(yb + int64_t(i) * p.y_sr + d0);
      const float* ibr = p.ibar + (int64_t(bh) * p.TQ + i) * D + d0;
#pragma unroll
      for (int e = 0; e < EPC; e += 4) {
        const float4 f = *reinterpret_cast<const float4*>(ibr + e);
        ibv[e] = f.x; ibv[e + 1] = f.y; ibv[e + 2] = f.z; ibv[e + 3] = f.w;
      }
      gi = p.g[int64_t(bh) * p.TQ + i];
    } else {
#pragma unroll
      for (int e = 0; e < EPC; ++e) ibv[e] = 0.f;
    }
    if constexpr (!LEAN) kreg[c] = ck;
    const T* eq = reinterpret_cast<const T*>(&cq);
    const T* ek = reinterpret_cast<const T*>(&ck);
    const T* ev = reinterpret_cast<const T*>(&cv);
    const T* ey = reinterpret_cast<const T*>(&cy);
    float dgate = 0.f, delta = 0.f, uii = 0.f;
    Chunk cd;
    T* ed = reinterpret_cast<T*>(&cd);
#pragma unroll
    for (int e = 0; e < EPC; ++e) {
      const float vy = E::to_f(ey[e]);
      const float dib = gi * vy;
      dgate += vy * (ibv[e] - E::to_f(ev[e]));
      delta += dib * ibv[e];
      uii += E::to_f(eq[e]) * E::to_f(ek[e]);
      // dI-bar in the operand dtype, as the reference stores it for its dots (flash_relation.py:215-216)
      ed[e] = E::from_f(dib);
    }
    part[0][r][cc] = dgate;
    part[1][r][cc] = delta;
    part[2][r][cc] = uii;
    if constexpr (!LEAN) {
      store_chunk(&sq[r * LD + d0], cq);
      store_chunk(&sd[r * LD + d0], cd);
      store_chunk(wq + r * DP + d0, cq);
    }
    store_chunk(wd + r * DP + d0, cd);
  }
  __syncthreads();
  // per-row terms
  if (tid < kRowBlock) {
    const int r = tid, i = i0 + r;
    const bool valid = i < p.TQ;
    float dgate = 0.f, delta = 0.f, uii = 0.f;
#pragma unroll
    for (int cc = 0; cc < CPR; ++cc) {
      dgate += part[0][r][cc];
      delta += part[1][r][cc];
      uii += part[2][r][cc];
    }
    float gi = 0.f, lse = kNegInf;
    if (valid) {
      gi = p.g[int64_t(bh) * p.TQ + i];
      lse = p.lse[int64_t(bh) * p.TQ + i];
    }
    const float da = dgate * gi * (1.0f - gi);
    const float s = sigmoid_acc(uii * p.scale * p.tau_inv);
    const float du = valid ? (-da) * s * (1.0f - s) * p.tau_inv : 0.f;
    const bool has = valid && lse > kNegInf;
    const int64_t w = int64_t(bh) * p.TQp + i;
    const float l2 = has ? lse * kLog2e : __builtin_inff();
    const float cv = valid ? da - delta : 0.f;
    if constexpr (LEAN) {
      float* st = p.stat + (int64_t(bh) * (p.TQp / kRowBlock) + blockIdx.x) * 128;
      st[r] = l2;
      st[64 + r] = cv;
    } else {
      p.lse2[w] = l2;
      p.cvec[w] = cv;
    }
    p.duii[w] = du;
    sdu[r] = du;
    sred[r] = valid ? -da * logf((float)(p.q_start + i) + 1.0f) : 0.f;
  }
  __syncthreads();
  // pass 2: dP1 accumulator initialised with the Self part dU_ii P2_i / sqrt(D)
#pragma unroll
  for (int c = 0; c < (LEAN ? 0 : CT); ++c) {
    const int idx = tid + 256 * c;
    if (idx >= NCH) break;
    const int r = idx / CPR, cc = idx % CPR;
    const int i = i0 + r;
    const int d0 = cc * EPC;
    if (i >= p.TQ || d0 >= D) continue;
    const float f = sdu[r] * p.scale;
    const T* ek = reinterpret_cast<const T*>(&kreg[c]);
    float* acc = p.dp1acc + (int64_t(bh) * p.TQ + i) * D + d0;
#pragma unroll
    for (int e = 0; e < EPC; e += 4)
      *reinterpret_cast<float4*>(acc + e) =
          make_float4(f * E::to_f(ek[e]), f * E::to_f(ek[e + 1]), f * E::to_f(ek[e + 2]), f * E::to_f(ek[e + 3]));
  }
  // transposed copies: row d holds the 64 rows of this block
  if constexpr (!LEAN) {
    T* wqT = reinterpret_cast<T*>(p.wqT) + int64_t(bh) * DP * p.TQp + i0;
    T* wdT = reinterpret_cast<T*>(p.wdibT) + int64_t(bh) * DP * p.TQp + i0;
    constexpr int CH = DP * kRowBlock / EPC;
    for (int c = tid; c < CH; c += 256) {
      const int d = c / (kRowBlock / EPC), cc = c % (kRowBlock / EPC);
      Chunk vq, vd;
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        if constexpr (sizeof(T) == 2) {
          const int r0 = (cc * 8 + 2 * w) * LD + d;
          vq.w[w] = uint32_t(sq[r0]) | (uint32_t(sq[r0 + LD]) << 16);
          vd.w[w] = uint32_t(sd[r0]) | (uint32_t(sd[r0 + LD]) << 16);
        } else {
          const int r0 = (cc * 4 + w) * LD + d;
          vq.w[w] = __float_as_uint(sq[r0]);
          vd.w[w] = __float_as_uint(sd[r0]);
        }
      }
      store_chunk(wqT + int64_t(d) * p.TQp + cc * EPC, vq);
      store_chunk(wdT + int64_t(d) * p.TQp + cc * EPC, vd);
    }
  }
  // dlam partial of this block: fixed-order tree over the 64 rows
  if (tid < 32) {
    float v = sred[tid] + sred[tid + 32];
#pragma unroll
    for (int m = 16; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
    if (tid == 0) p.dlam_part[int64_t(bh) * (p.TQp / kRowBlock) + blockIdx.x] = v;
  }
}

// ------------------------------------------------------------------------------------------------
// 2. key blocks
// ------------------------------------------------------------------------------------------------
// Transposed staging of a [64 keys x DP] block into LDS as [DP][LDT] (head-dim major):
// item = 4 consecutive keys x one 16-byte chunk of the head dim.
template <typename T, int DP, int NTH>
__device__ __forceinline__ void stage_transposed(T* dst, int LDT, const T* base, int64_t row_stride, int j0, int nrows,
                                                 int D, int tid) {
  constexpr int EPC = 16 / sizeof(T);
  constexpr int ITEMS = (64 / 4) * (DP / EPC);
  for (int it = tid; it < ITEMS; it += NTH) {
    const int kq = it % 16, cc = it / 16;
    Chunk v[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int j = j0 + 4 * kq + r;
      v[r] = (j < nrows && cc * EPC < D) ? load_chunk(base + int64_t(j) * row_stride + cc * EPC) : zero_chunk();
    }
    if constexpr (sizeof(T) == 2) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int w = e >> 1, sh = (e & 1) * 16;
        uint2 o;
        o.x = ((v[0].w[w] >> sh) & 0xffffu) | (((v[1].w[w] >> sh) & 0xffffu) << 16);
        o.y = ((v[2].w[w] >> sh) & 0xffffu) | (((v[3].w[w] >> sh) & 0xffffu) << 16);
        *reinterpret_cast<uint2*>(&dst[(cc * 8 + e) * LDT + 4 * kq]) = o;
      }
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        uint4 o;
        o.x = v[0].w[e];
        o.y = v[1].w[e];
        o.z = v[2].w[e];
        o.w = v[3].w[e];
        *reinterpret_cast<uint4*>(&dst[(cc * 4 + e) * LDT + 4 * kq]) = o;
      }
    }
  }
}

template <typename T, int DP, int BM, bool WITH_DQ>
__global__ void __launch_bounds__(256) bwd_keys_kernel(const BwdParams p) {
  using E = Elem<T>;
  using Frag = typename E::Frag;
  constexpr int BN = 64;
  constexpr int KS = DP / 32;
  constexpr int DT = DP / 16;
  constexpr int QT = BM / 16;           // query tiles per block
  constexpr int EPC = 16 / sizeof(T);
  constexpr int PADE = 16 / sizeof(T);  // 16-byte row padding
  constexpr int QLD = DP + PADE;        // Qs / Ds row stride
  constexpr int TLD = BM + (sizeof(T) == 2 ? 8 : 4);   // QTs / DTs row stride
  constexpr int ULD = BN + PADE;        // dUs row stride
  constexpr int KLD = BN + PADE;        // KTs row stride
  __shared__ __align__(16) T Qs[BM * QLD];
  __shared__ __align__(16) T Ds[BM * QLD];
  __shared__ __align__(16) T QTs[DP * TLD];
  __shared__ __align__(16) T DTs[DP * TLD];
  __shared__ __align__(16) T dUs[WITH_DQ ? BM * ULD : 1];
  __shared__ __align__(16) T KTs[WITH_DQ ? DP * KLD : 1];
  __shared__ __align__(16) float Ls[BM];
  __shared__ __align__(16) float Cs[BM];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int li = lane & 15, lg = lane >> 4;
  const int BH = p.B * p.H;
  const int bh = blockIdx.x % BH;
  const int kb = blockIdx.x / BH;
  const int b = bh / p.H, h = bh % p.H;
  const int k0 = kb * BN;
  const int D = p.D;
  const T* kbase = reinterpret_cast<const T*>(p.p2) + b * p.k_sb + h * p.k_sh;
  const T* vbase = reinterpret_cast<const T*>(p.info) + b * p.v_sb + h * p.v_sh;

  // this wave's 16 keys as B fragments (k = head dim, column = key)
  const int jw = k0 + 16 * wave + li;
  Frag kf[KS], vf[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    const int d0 = 32 * ks + 8 * lg;
    if (jw < p.TK && d0 < D) {
      kf[ks] = E::load8(kbase + int64_t(jw) * p.k_sr + d0);
      vf[ks] = E::load8(vbase + int64_t(jw) * p.v_sr + d0);
    } else {
      kf[ks] = E::zero();
      vf[ks] = E::zero();
    }
  }
  if constexpr (WITH_DQ) stage_transposed<T, DP, 256>(KTs, KLD, kbase, p.k_sr, k0, p.TK, D, tid);

  const int nqb = p.TQp / BM;
  const int qb_lo = max(0, k0 + 1 - p.q_start) / BM;
  const T* wq = reinterpret_cast<const T*>(p.wq) + int64_t(bh) * p.TQp * DP;
  const T* wd = reinterpret_cast<const T*>(p.wdib) + int64_t(bh) * p.TQp * DP;
  const T* wqT = reinterpret_cast<const T*>(p.wqT) + int64_t(bh) * DP * p.TQp;
  const T* wdT = reinterpret_cast<const T*>(p.wdibT) + int64_t(bh) * DP * p.TQp;
  const float* lse2 = p.lse2 + int64_t(bh) * p.TQp;
  const float* cvec = p.cvec + int64_t(bh) * p.TQp;

  // staging: rows (Q, dI-bar) and transposed (Q^T, dI-bar^T) blocks, plus lse2 / c
  constexpr int RCH = BM * DP / EPC;      // row chunks per array
  constexpr int RCT = (RCH + 255) / 256;
  constexpr int TCH = DP * BM / EPC;      // transposed chunks per array
  constexpr int TCT = (TCH + 255) / 256;
  Chunk rq[RCT], rd[RCT], tq[TCT], td[TCT];
  float sl = 0.f, sc = 0.f;
  auto prefetch = [&](int qb) {
    const int i0 = qb * BM;
#pragma unroll
    for (int c = 0; c < RCT; ++c) {
      const int idx = tid + 256 * c;
      if (idx < RCH) {
        const int r = idx / (DP / EPC), cc = idx % (DP / EPC);
        rq[c] = load_chunk(wq + int64_t(i0 + r) * DP + cc * EPC);
        rd[c] = load_chunk(wd + int64_t(i0 + r) * DP + cc * EPC);
      }
    }
#pragma unroll
    for (int c = 0; c < TCT; ++c) {
      const int idx = tid + 256 * c;
      if (idx < TCH) {
        const int d = idx / (BM / EPC), cc = idx % (BM / EPC);
        tq[c] = load_chunk(wqT + int64_t(d) * p.TQp + i0 + cc * EPC);
        td[c] = load_chunk(wdT + int64_t(d) * p.TQp + i0 + cc * EPC);
      }
    }
    if (tid < BM) {
      sl = lse2[i0 + tid];
      sc = cvec[i0 + tid];
    }
  };
  auto commit = [&]() {
#pragma unroll
    for (int c = 0; c < RCT; ++c) {
      const int idx = tid + 256 * c;
      if (idx < RCH) {
        const int r = idx / (DP / EPC), cc = idx % (DP / EPC);
        store_chunk(&Qs[r * QLD + cc * EPC], rq[c]);
        store_chunk(&Ds[r * QLD + cc * EPC], rd[c]);
      }
    }
#pragma unroll
    for (int c = 0; c < TCT; ++c) {
      const int idx = tid + 256 * c;
      if (idx < TCH) {
        const int d = idx / (BM / EPC), cc = idx % (BM / EPC);
        store_chunk(&QTs[d * TLD + cc * EPC], tq[c]);
        store_chunk(&DTs[d * TLD + cc * EPC], td[c]);
      }
    }
    if (tid < BM) {
      Ls[tid] = sl;
      Cs[tid] = sc;
    }
  };

  f32x4 dvacc[DT], dkacc[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) {
    dvacc[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
    dkacc[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  const float c2 = p.scale * kLog2e;

  if (qb_lo < nqb) prefetch(qb_lo);
  for (int qb = qb_lo; qb < nqb; ++qb) {
    __syncthreads();
    commit();
    __syncthreads();
    if (qb + 1 < nqb) prefetch(qb + 1);
    const int i0 = qb * BM;
    const bool masked = p.q_start + i0 <= k0 + BN - 1;

    // U = Q K^T and dW = dI-bar V^T: rows = queries, columns = this wave's keys
    f32x4 sacc[QT], wacc[QT];
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
      sacc[qt] = f32x4{0.f, 0.f, 0.f, 0.f};
      wacc[qt] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
#pragma unroll
      for (int qt = 0; qt < QT; ++qt) {
        const Frag aq = E::load8(&Qs[(16 * qt + li) * QLD + 32 * ks + 8 * lg]);
        sacc[qt] = E::mma(aq, kf[ks], sacc[qt]);
        const Frag ad = E::load8(&Ds[(16 * qt + li) * QLD + 32 * ks + 8 * lg]);
        wacc[qt] = E::mma(ad, vf[ks], wacc[qt]);
      }
    }
    // w and dU per (query 16qt + 4lg + r, key jw)
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
      const float4 l4 = *reinterpret_cast<const float4*>(&Ls[16 * qt + 4 * lg]);
      const float4 c4 = *reinterpret_cast<const float4*>(&Cs[16 * qt + 4 * lg]);
      const float lv[4] = {l4.x, l4.y, l4.z, l4.w};
      const float cv[4] = {c4.x, c4.y, c4.z, c4.w};
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float u2 = sacc[qt][r] * c2;  // U in log2 units
        const float sg = frcp(1.0f + fexp2(-u2));
        float w = fexp2(u2 * sg - lv[r]);
        if (masked) {
          const int qa = p.q_start + i0 + 16 * qt + 4 * lg + r;
          if (jw >= qa) w = 0.f;
        }
        const float u = sacc[qt][r] * p.scale;
        const float de = w * (wacc[qt][r] + cv[r]);
        const float du = de * (sg * (1.0f + u * (1.0f - sg)));
        sacc[qt][r] = w;
        wacc[qt][r] = du;
      }
    }
    // dV += W^T dI-bar, dK += dU^T Q  (k = queries, permuted order 4lg + r | 16 + 4lg + r)
#pragma unroll
    for (int kk = 0; kk < QT / 2; ++kk) {
      float wv[8], uv[8];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        wv[r] = sacc[2 * kk][r];
        wv[4 + r] = sacc[2 * kk + 1][r];
        uv[r] = wacc[2 * kk][r];
        uv[4 + r] = wacc[2 * kk + 1][r];
      }
      const Frag aw = E::from_f32(wv);
      const Frag au = E::from_f32(uv);
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const T* drow = &DTs[(16 * dt + li) * TLD + 32 * kk + 4 * lg];
        dvacc[dt] = E::mma(aw, E::load4x2(drow, drow + 16), dvacc[dt]);
        const T* qrow = &QTs[(16 * dt + li) * TLD + 32 * kk + 4 * lg];
        dkacc[dt] = E::mma(au, E::load4x2(qrow, qrow + 16), dkacc[dt]);
      }
    }
    if constexpr (WITH_DQ) {
      // dU -> LDS as [query][key], then dQ = dU K over the workgroup's 64 keys
#pragma unroll
      for (int qt = 0; qt < QT; ++qt)
#pragma unroll
        for (int r = 0; r < 4; ++r) dUs[(16 * qt + 4 * lg + r) * ULD + 16 * wave + li] = E::from_f(wacc[qt][r]);
      __syncthreads();
      for (int tile = wave; tile < QT * DT; tile += 4) {
        const int qt = tile / DT, dt = tile % DT;
        f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kk = 0; kk < BN / 32; ++kk) {
          const Frag a = E::load8(&dUs[(16 * qt + li) * ULD + 32 * kk + 8 * lg]);
          const Frag bk = E::load8(&KTs[(16 * dt + li) * KLD + 32 * kk + 8 * lg]);
          acc = E::mma(a, bk, acc);
        }
        const int d = 16 * dt + li;
        if (d < D) {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int i = i0 + 16 * qt + 4 * lg + r;
            if (i < p.TQ) unsafeAtomicAdd(&p.dp1acc[(int64_t(bh) * p.TQ + i) * D + d], acc[r] * p.scale);
          }
        }
      }
    }
  }

  // Self terms of key rows that are also queries, then the single store of dP2 and dI~
  const T* q = reinterpret_cast<const T*>(p.p1) + b * p.q_sb + h * p.q_sh;
  const T* dy = reinterpret_cast<const T*>(p.dy) + b * p.y_sb + h * p.y_sh;
  T* dk = reinterpret_cast<T*>(p.dp2) + b * p.dk_sb + h * p.dk_sh;
  T* dv = reinterpret_cast<T*>(p.dinfo) + b * p.dv_sb + h * p.dv_sh;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int j = k0 + 16 * wave + 4 * lg + r;
    if (j >= p.TK) continue;
    const int i = j - p.q_start;
    float gs = 0.f, us = 0.f;
    if (i >= 0) {
      gs = p.g[int64_t(bh) * p.TQ + i];
      us = p.duii[int64_t(bh) * p.TQp + i];
    }
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      const int d = 16 * dt + li;
      if (d >= D) continue;
      float vv = dvacc[dt][r], kk = dkacc[dt][r];
      if (i >= 0) {
        vv += (1.0f - gs) * E::to_f(dy[int64_t(i) * p.y_sr + d]);
        kk += us * E::to_f(q[int64_t(i) * p.q_sr + d]);
      }
      dv[int64_t(j) * p.dv_sr + d] = E::from_f(vv);
      dk[int64_t(j) * p.dk_sr + d] = E::from_f(kk * p.scale);
    }
  }
}

// ------------------------------------------------------------------------------------------------
// 3a. one-pass: fp32 dP1 accumulator -> output
// ------------------------------------------------------------------------------------------------
template <typename T>
__global__ void __launch_bounds__(256) bwd_dp1_out_kernel(const BwdParams p) {
  const int64_t n = int64_t(p.B) * p.H * p.TQ * p.D;
  for (int64_t e = blockIdx.x * 256ll + threadIdx.x; e < n; e += int64_t(gridDim.x) * 256) {
    const int d = int(e % p.D);
    const int64_t rrow = e / p.D;
    const int i = int(rrow % p.TQ);
    const int bh = int(rrow / p.TQ);
    const int b = bh / p.H, h = bh % p.H;
    T* o = reinterpret_cast<T*>(p.dp1) + b * p.dq_sb + h * p.dq_sh + int64_t(i) * p.dq_sr;
    o[d] = Elem<T>::from_f(p.dp1acc[e]);
  }
}

// ------------------------------------------------------------------------------------------------
// 3b. deterministic: query-stationary dQ (same staging and layouts as the forward kernel)
// ------------------------------------------------------------------------------------------------
template <typename T, int DP, int BN>
__global__ void __launch_bounds__(128) bwd_queries_kernel(const BwdParams p) {
  using E = Elem<T>;
  using Frag = typename E::Frag;
  constexpr int NW = 2, NTH = 128, BM = 64;
  constexpr int KS = DP / 32, DT = DP / 16, NT = BN / 16;
  constexpr int EPC = 16 / sizeof(T);
  constexpr int KLD = DP + EPC;
  constexpr int TLD = BN + (sizeof(T) == 2 ? 8 : 4);
  constexpr int CPR = DP / EPC;
  constexpr int KCH = BN * CPR;
  __shared__ __align__(16) T Ks[BN * KLD];
  __shared__ __align__(16) T Vs[BN * KLD];
  __shared__ __align__(16) T KTs[DP * TLD];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int li = lane & 15, lg = lane >> 4;
  const int BH = p.B * p.H;
  const int bh = blockIdx.x % BH;
  const int nqb = (p.TQ + BM - 1) / BM;
  const int qb = nqb - 1 - blockIdx.x / BH;
  const int b = bh / p.H, h = bh % p.H;
  const int D = p.D;
  const T* kbase = reinterpret_cast<const T*>(p.p2) + b * p.k_sb + h * p.k_sh;
  const T* vbase = reinterpret_cast<const T*>(p.info) + b * p.v_sb + h * p.v_sh;
  const T* wq = reinterpret_cast<const T*>(p.wq) + int64_t(bh) * p.TQp * DP;
  const T* wd = reinterpret_cast<const T*>(p.wdib) + int64_t(bh) * p.TQp * DP;

  const int q0 = qb * BM + 32 * wave;
  Frag qf[2][KS], df[2][KS];
  float lse2[2], cv[2];
  int qabs[2];
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    const int qi = q0 + 16 * s + li;  // < TQp: the copies are padded with zero rows
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      qf[s][ks] = E::load8(wq + int64_t(qi) * DP + 32 * ks + 8 * lg);
      df[s][ks] = E::load8(wd + int64_t(qi) * DP + 32 * ks + 8 * lg);
    }
    lse2[s] = p.lse2[int64_t(bh) * p.TQp + qi];
    cv[s] = p.cvec[int64_t(bh) * p.TQp + qi];
    qabs[s] = p.q_start + qi;
  }
  const int qlast = min(p.TQ, (qb + 1) * BM) - 1;
  const int kend = p.q_start + qlast;
  const int nkb = (kend + BN - 1) / BN;
  const bool wave_active = q0 < p.TQ;
  const int wave_kend = wave_active ? p.q_start + min(q0 + 32, p.TQ) - 1 : 0;
  const float c2 = p.scale * kLog2e;

  f32x4 dq[DT][2];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int s = 0; s < 2; ++s) dq[dt][s] = f32x4{0.f, 0.f, 0.f, 0.f};

  for (int kb = 0; kb < nkb; ++kb) {
    const int j0 = kb * BN;
    __syncthreads();
    for (int idx = tid; idx < KCH; idx += NTH) {
      const int row = idx / CPR, cc = idx % CPR;
      const int j = j0 + row;
      const bool ok = j < p.TK && cc * EPC < D;
      store_chunk(&Ks[row * KLD + cc * EPC], ok ? load_chunk(kbase + int64_t(j) * p.k_sr + cc * EPC) : zero_chunk());
      store_chunk(&Vs[row * KLD + cc * EPC], ok ? load_chunk(vbase + int64_t(j) * p.v_sr + cc * EPC) : zero_chunk());
    }
    if constexpr (BN == 64) {
      stage_transposed<T, DP, NTH>(KTs, TLD, kbase, p.k_sr, j0, p.TK, D, tid);
    } else {
      // 32-key blocks (fp32): the same transposed staging over 32 rows
      constexpr int ITEMS = (BN / 4) * (DP / EPC);
      for (int it = tid; it < ITEMS; it += NTH) {
        const int kq = it % (BN / 4), cc = it / (BN / 4);
        Chunk v[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int j = j0 + 4 * kq + r;
          v[r] = (j < p.TK && cc * EPC < D) ? load_chunk(kbase + int64_t(j) * p.k_sr + cc * EPC) : zero_chunk();
        }
#pragma unroll
        for (int e = 0; e < EPC; ++e) {
          if constexpr (sizeof(T) == 4) {
            uint4 o;
            o.x = v[0].w[e]; o.y = v[1].w[e]; o.z = v[2].w[e]; o.w = v[3].w[e];
            *reinterpret_cast<uint4*>(&KTs[(cc * 4 + e) * TLD + 4 * kq]) = o;
          } else {
            const int w = e >> 1, sh = (e & 1) * 16;
            uint2 o;
            o.x = ((v[0].w[w] >> sh) & 0xffffu) | (((v[1].w[w] >> sh) & 0xffffu) << 16);
            o.y = ((v[2].w[w] >> sh) & 0xffffu) | (((v[3].w[w] >> sh) & 0xffffu) << 16);
            *reinterpret_cast<uint2*>(&KTs[(cc * 8 + e) * TLD + 4 * kq]) = o;
          }
        }
      }
    }
    __syncthreads();
    if (!wave_active || j0 >= wave_kend) continue;
    const bool masked = j0 + BN > p.q_start + q0;
    f32x4 sacc[NT][2], wacc[NT][2];
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        sacc[t][s] = f32x4{0.f, 0.f, 0.f, 0.f};
        wacc[t][s] = f32x4{0.f, 0.f, 0.f, 0.f};
      }
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const Frag ak = E::load8(&Ks[(16 * t + li) * KLD + 32 * ks + 8 * lg]);
        const Frag av = E::load8(&Vs[(16 * t + li) * KLD + 32 * ks + 8 * lg]);
#pragma unroll
        for (int s = 0; s < 2; ++s) {
          sacc[t][s] = E::mma(ak, qf[s][ks], sacc[t][s]);
          wacc[t][s] = E::mma(av, df[s][ks], wacc[t][s]);
        }
      }
    }
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float u2 = sacc[t][s][r] * c2;
          const float sg = frcp(1.0f + fexp2(-u2));
          float w = fexp2(u2 * sg - lse2[s]);
          if (masked) {
            const int j = j0 + 16 * t + 4 * lg + r;
            if (j >= qabs[s]) w = 0.f;
          }
          const float u = sacc[t][s][r] * p.scale;
          const float de = w * (wacc[t][s][r] + cv[s]);
          sacc[t][s][r] = de * (sg * (1.0f + u * (1.0f - sg)));
        }
    // dQ^T += K^T dU^T
#pragma unroll
    for (int kk = 0; kk < NT / 2; ++kk) {
      Frag bu[2];
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        float uv[8];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          uv[r] = sacc[2 * kk][s][r];
          uv[4 + r] = sacc[2 * kk + 1][s][r];
        }
        bu[s] = E::from_f32(uv);
      }
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const T* krow = &KTs[(16 * dt + li) * TLD + 32 * kk + 4 * lg];
        const Frag ak = E::load4x2(krow, krow + 16);
#pragma unroll
        for (int s = 0; s < 2; ++s) dq[dt][s] = E::mma(ak, bu[s], dq[dt][s]);
      }
    }
  }
  if (!wave_active) return;
  T* out = reinterpret_cast<T*>(p.dp1) + b * p.dq_sb + h * p.dq_sh;
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    const int qi = q0 + 16 * s + li;
    if (qi >= p.TQ) continue;
    const float* init = p.dp1acc + (int64_t(bh) * p.TQ + qi) * D;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int d = 16 * dt + 4 * lg + r;
        if (d < D) out[int64_t(qi) * p.dq_sr + d] = E::from_f(dq[dt][s][r] * p.scale + init[d]);
      }
  }
}

__global__ void __launch_bounds__(256) bwd_zero_rows_kernel(mote_view v, int H, int rows, int D, int es) {
  const int b = blockIdx.x / H, h = blockIdx.x % H;
  char* base = reinterpret_cast<char*>(v.data) + (b * v.stride_b + h * v.stride_h) * es;
  for (int e = threadIdx.x; e < rows * D; e += 256) {
    char* q = base + (int64_t(e / D) * v.stride_r + e % D) * es;
    if (es == 2) *reinterpret_cast<uint16_t*>(q) = 0;
    else *reinterpret_cast<float*>(q) = 0.f;
  }
}

__global__ void __launch_bounds__(256) bwd_dlam_kernel(const float* part, int n, float* out) {
  __shared__ float red[256];
  dlam_sum(part, n, out, red);
}

// ------------------------------------------------------------------------------------------------
// host side
// ------------------------------------------------------------------------------------------------
struct WsLayout {
  size_t wq, wdib, wqT, wdibT, lse2, cvec, stat, dut, kvq, duii, dp1acc, dlam_part, total;
};

static size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

// Whether the tile path's key and query work share one launch (bwd_kvq_kernel): by default always.
// Against the two launches (event timing over whole backward calls, rows stage included) it measured
// as fast or faster at every shape tried from one key block to C3: C3 162-174 against 175-200 us,
// B 4 x H 8 at 658 rows 32.7 against 36.0 us, H 8 at 2048 rows 68 against 79 us, H 16 at 1024 rows
// (dh 64) 37 against 42 us; within 0.5 us at 300 rows and at one key block. The environment
// variable MOTE_BWD_FUSED = 0 selects the two launches (1 the one launch, the default). It is read
// on every call (a few hundred ns against tens of microseconds of launches).
static bool fused_bwd_wanted(const mote_relation_bwd_args* a) {
  (void)a;
  const char* e = getenv("MOTE_BWD_FUSED");
  return !(e && e[0] == '0');
}

// bf16 with a head dim the tile kernels are compiled for: the atomic-free tile path.
static bool use_tiles(const mote_relation_bwd_args* a) {
  return a->dtype == MOTE_BF16 && padded_dim(a->D) == a->D && tile_strides_ok(a->p1, a->p2, a->info);
}

static WsLayout ws_layout(const mote_relation_bwd_args* a) {
  const size_t es = a->dtype == MOTE_BF16 ? 2 : 4;
  const size_t BH = size_t(a->B) * a->H;
  const size_t TQp = size_t((a->TQ + kRowBlock - 1) / kRowBlock) * kRowBlock;
  const size_t DP = padded_dim(a->D);
  const bool tiles = use_tiles(a);
  WsLayout w{};
  size_t o = 0;
  w.wdib = o; o = align256(o + BH * TQp * DP * es);
  if (tiles) {
    w.stat = o; o = align256(o + BH * (TQp / kRowBlock) * 128 * 4);
    // dU fragments: 8 KB per visible (query block, key block) pair
    w.dut = o; o = align256(o + BH * size_t(PairTable::total(a->TQ, a->q_start)) * 8192);
    w.kvq = o; o = align256(o + (kKvqCounts + BH * (TQp / kRowBlock)) * 4);
  } else {
    w.wq = o; o = align256(o + BH * TQp * DP * es);
    w.wqT = o; o = align256(o + BH * TQp * DP * es);
    w.wdibT = o; o = align256(o + BH * TQp * DP * es);
    w.lse2 = o; o = align256(o + BH * TQp * 4);
    w.cvec = o; o = align256(o + BH * TQp * 4);
    w.dp1acc = o; o = align256(o + BH * size_t(a->TQ) * a->D * 4);
  }
  w.duii = o; o = align256(o + BH * TQp * 4);
  w.dlam_part = o; o = align256(o + BH * (TQp / kRowBlock) * 4);
  w.total = o;
  return w;
}

size_t bwd_workspace_bytes(const mote_relation_bwd_args* a) { return ws_layout(a).total; }

// Register-staged kernels (fp32, and bf16 head dims that need padding).
template <typename T, int DP>
static void launch_bwd_t(const BwdParams& p, bool deterministic, int stages, hipStream_t stream) {
  const int BH = p.B * p.H;
  if (stages & MOTE_BWD_ROWS)
    hipLaunchKernelGGL((bwd_rows_kernel<T, DP, false>), dim3(p.TQp / kRowBlock, BH), dim3(256), 0, stream, p);
  const int nkb = (p.TK + 63) / 64;
  constexpr int BM = sizeof(T) == 2 ? 64 : 32;
  if (stages & MOTE_BWD_KEYS) {
    if (!deterministic)
      hipLaunchKernelGGL((bwd_keys_kernel<T, DP, BM, true>), dim3(nkb * BH), dim3(256), 0, stream, p);
    else
      hipLaunchKernelGGL((bwd_keys_kernel<T, DP, BM, false>), dim3(nkb * BH), dim3(256), 0, stream, p);
  }
  if ((stages & MOTE_BWD_QUERIES) && deterministic) {
    constexpr int BNQ = sizeof(T) == 2 ? 64 : 32;
    const int nqb = (p.TQ + 63) / 64;
    hipLaunchKernelGGL((bwd_queries_kernel<T, DP, BNQ>), dim3(nqb * BH), dim3(128), 0, stream, p);
  }
  if (stages & MOTE_BWD_FINISH) {
    if (!deterministic) {
      const int64_t n = int64_t(BH) * p.TQ * p.D;
      const int blocks = int((n + 255) / 256 < 4096 ? (n + 255) / 256 : 4096);
      hipLaunchKernelGGL((bwd_dp1_out_kernel<T>), dim3(blocks), dim3(256), 0, stream, p);
    }
    hipLaunchKernelGGL(bwd_dlam_kernel, dim3(1), dim3(256), 0, stream, p.dlam_part, BH * (p.TQp / kRowBlock), p.dlam);
  }
}

// dlam is summed by the last workgroup of the query-stationary kernel (MOTE_BWD_QUERIES): the finish
// stage has nothing left to do on this path.
template <int DP>
static void launch_bwd_tile_path(const BwdParams& p, int stages, hipStream_t stream) {
  const int BH = p.B * p.H;
  if (stages & MOTE_BWD_ROWS)
    hipLaunchKernelGGL((bwd_rows_kernel<bf16_t, DP, true>), dim3(p.TQp / kRowBlock, BH), dim3(256), 0, stream, p);
  launch_bwd_tiles(p, stages, stream);
}

int launch_bwd(const mote_relation_bwd_args* a, hipStream_t stream) {
  if (!a) return set_error(MOTE_ERR_ARGUMENT, "relation_bwd: null args");
  if (a->dtype != MOTE_F32 && a->dtype != MOTE_BF16) return set_error(MOTE_ERR_ARGUMENT, "relation_bwd: bad dtype %d", a->dtype);
  if (a->D <= 0 || a->D > 128 || a->D % 8 != 0)
    return set_error(MOTE_ERR_SHAPE, "relation_bwd: head dim %d unsupported (need 8 <= D <= 128, D %% 8 == 0)", a->D);
  if (a->B <= 0 || a->H <= 0 || a->TQ < 0 || a->TK != a->q_start + a->TQ)
    return set_error(MOTE_ERR_SHAPE, "relation_bwd: bad sizes (TK=%d, q_start=%d, TQ=%d)", a->TK, a->q_start, a->TQ);
  if (!a->dlam) return set_error(MOTE_ERR_ARGUMENT, "relation_bwd: null dlam");
  const WsLayout w = ws_layout(a);
  if (a->TQ == 0) {
    // no query rows: dP2 / dI~ of the prefix and dlam are zero (fill kernels, no memset nodes)
    const int es = a->dtype == MOTE_BF16 ? 2 : 4;
    const int BH = a->B * a->H;
    if (a->TK > 0) {
      hipLaunchKernelGGL(bwd_zero_rows_kernel, dim3(BH), dim3(256), 0, stream, a->dp2, a->H, a->TK, a->D, es);
      hipLaunchKernelGGL(bwd_zero_rows_kernel, dim3(BH), dim3(256), 0, stream, a->dinfo, a->H, a->TK, a->D, es);
    }
    hipLaunchKernelGGL(bwd_dlam_kernel, dim3(1), dim3(256), 0, stream, (const float*)nullptr, 0, a->dlam);
    return check_launch("relation_bwd (empty)");
  }
  if (!a->p1.data || !a->p2.data || !a->info.data || !a->dy.data || !a->ibar || !a->lse || !a->g || !a->dp1.data ||
      !a->dp2.data || !a->dinfo.data)
    return set_error(MOTE_ERR_ARGUMENT, "relation_bwd: null tensor pointer");
  if (!a->workspace || a->workspace_bytes < w.total)
    return set_error(MOTE_ERR_WORKSPACE, "relation_bwd: workspace of %zu bytes, %zu needed", a->workspace_bytes, w.total);
  BwdParams p{};
  p.p1 = a->p1.data; p.q_sb = a->p1.stride_b; p.q_sh = a->p1.stride_h; p.q_sr = a->p1.stride_r;
  p.p2 = a->p2.data; p.k_sb = a->p2.stride_b; p.k_sh = a->p2.stride_h; p.k_sr = a->p2.stride_r;
  p.info = a->info.data; p.v_sb = a->info.stride_b; p.v_sh = a->info.stride_h; p.v_sr = a->info.stride_r;
  p.dy = a->dy.data; p.y_sb = a->dy.stride_b; p.y_sh = a->dy.stride_h; p.y_sr = a->dy.stride_r;
  p.ibar = a->ibar; p.lse = a->lse; p.g = a->g;
  p.dp1 = a->dp1.data; p.dq_sb = a->dp1.stride_b; p.dq_sh = a->dp1.stride_h; p.dq_sr = a->dp1.stride_r;
  p.dp2 = a->dp2.data; p.dk_sb = a->dp2.stride_b; p.dk_sh = a->dp2.stride_h; p.dk_sr = a->dp2.stride_r;
  p.dinfo = a->dinfo.data; p.dv_sb = a->dinfo.stride_b; p.dv_sh = a->dinfo.stride_h; p.dv_sr = a->dinfo.stride_r;
  p.dlam = a->dlam;
  const bool tiles = use_tiles(a);
  char* ws = reinterpret_cast<char*>(a->workspace);
  p.wdib = ws + w.wdib;
  p.duii = reinterpret_cast<float*>(ws + w.duii);
  p.dlam_part = reinterpret_cast<float*>(ws + w.dlam_part);
  if (tiles) {
    p.stat = reinterpret_cast<float*>(ws + w.stat);
    p.dut = ws + w.dut;
    p.npairs = PairTable::total(a->TQ, a->q_start);
    // the fused key + query launch: head dims with two workgroups per CU, one (batch x head)'s pairs
    // addressable by a 32-bit buffer offset
    if (padded_dim(a->D) <= 96 && p.npairs * 8192 < (int64_t(1) << 31) && fused_bwd_wanted(a)) {
      p.kvq = reinterpret_cast<int*>(ws + w.kvq);
      const int BH = a->B * a->H;
      p.kvq_nq = BH % 8 == 0 ? 8 : BH % 4 == 0 ? 4 : BH % 2 == 0 ? 2 : 1;
      p.kvq_spin = kKvqSpinLimit;
      // a test of the give-up path: every wait's target out of reach, a few polls
      const char* u = getenv("MOTE_BWD_UNREACHABLE_WAIT");
      if (u && u[0] == '1') {
        p.kvq_extra = 1;
        p.kvq_spin = 4;
      }
    }
  } else {
    p.wq = ws + w.wq; p.wqT = ws + w.wqT; p.wdibT = ws + w.wdibT;
    p.lse2 = reinterpret_cast<float*>(ws + w.lse2);
    p.cvec = reinterpret_cast<float*>(ws + w.cvec);
    p.dp1acc = reinterpret_cast<float*>(ws + w.dp1acc);
  }
  p.B = a->B; p.H = a->H; p.TQ = a->TQ; p.TK = a->TK; p.D = a->D; p.q_start = a->q_start;
  p.TQp = (a->TQ + kRowBlock - 1) / kRowBlock * kRowBlock;
  p.scale = 1.0f / sqrtf((float)a->D);
  p.tau_inv = 1.0f / a->tau_s;
  const int DP = padded_dim(a->D);
  const bool det = a->deterministic != 0;
  const int st = a->stages ? a->stages : (MOTE_BWD_ROWS | MOTE_BWD_KEYS | MOTE_BWD_QUERIES | MOTE_BWD_FINISH);
  if (tiles) {
    switch (DP) {
      case 32: launch_bwd_tile_path<32>(p, st, stream); break;
      case 64: launch_bwd_tile_path<64>(p, st, stream); break;
      case 96: launch_bwd_tile_path<96>(p, st, stream); break;
      default: launch_bwd_tile_path<128>(p, st, stream); break;
    }
  } else if (a->dtype == MOTE_BF16) {
    switch (DP) {
      case 32: launch_bwd_t<bf16_t, 32>(p, det, st, stream); break;
      case 64: launch_bwd_t<bf16_t, 64>(p, det, st, stream); break;
      case 96: launch_bwd_t<bf16_t, 96>(p, det, st, stream); break;
      default: launch_bwd_t<bf16_t, 128>(p, det, st, stream); break;
    }
  } else {
    switch (DP) {
      case 32: launch_bwd_t<float, 32>(p, det, st, stream); break;
      case 64: launch_bwd_t<float, 64>(p, det, st, stream); break;
      case 96: launch_bwd_t<float, 96>(p, det, st, stream); break;
      default: launch_bwd_t<float, 128>(p, det, st, stream); break;
    }
  }
  return check_launch("relation_bwd");
}

}  // namespace mote
