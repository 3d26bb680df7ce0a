// Fused Relation forward for gfx950.
//
// One workgroup owns BM = 32 * NW query rows of one (sequence, head); wave w owns rows
// [32w, 32w + 32) as two 16-row tiles. The strictly-past keys are streamed in blocks of BN rows:
// each block of P2 is staged row-major in LDS (Ks) and the matching I~ block transposed (Vt, head
// dim major), both from registers prefetched during the previous block's math.
//
// Per block and wave:
//   S^T = K Q^T       A = K rows from Ks, B = the wave's queries (registers, loaded once)
//   e   = SiLU(S^T / sqrt(D)) in log2 units, masked on the diagonal blocks
//   online softmax over keys with a running max per query, rescaled only when a block raises it
//   by more than 2^8 (the reference's RESCALE_THRESH, flash_relation.py:57, 124-134)
//   O^T += V^T P^T    A = I~ columns from Vt, B = P^T taken straight from the S^T accumulators:
//                     a lane holds one query and keys 4g + r of each 16-key tile, which is a
//                     permuted k order of the operand; the Vt fragment uses the same order.
// Epilogue per query (flash_relation.py:151-183): LSE, I-bar = O / l, the Self score from the
// query's own key row, g = sigmoid(LSE - lam ln(i+1) - S), Y = (1 - g) I~_i + g I-bar.
//
// Block order: the grid is [query block (descending) x sequence x head], head fastest. Long
// query blocks are dispatched first (longest-processing-time order) and consecutive workgroups
// of one query block land on different XCDs, so with 8 heads every XCD's L2 holds one head's
// P2 / I~ rows.
#include <stdlib.h>
#include <type_traits>

#include "common.hpp"
#include "params.hpp"
#include "tiles.hpp"

namespace mote {

template <typename T, int DP, int BN, int NW>
__global__ void __launch_bounds__(NW * 64) relation_fwd_kernel(const FwdParams p) {
  using E = Elem<T>;
  using Frag = typename E::Frag;
  constexpr int NTH = NW * 64;
  constexpr int KS = DP / 32;                 // k-steps over the head dim
  constexpr int DT = DP / 16;                 // 16-row tiles of the head dim (outputs)
  constexpr int NT = BN / 16;                 // 16-key tiles per block
  constexpr int BM = NW * 32;
  constexpr int EPC = 16 / sizeof(T);         // elements per 16-byte chunk
  constexpr int KLD = DP + EPC;               // Ks row stride (elements): +16 bytes against bank conflicts
  constexpr int VLD = BN + (sizeof(T) == 2 ? 8 : 4);
  constexpr int CPR = DP / EPC;               // chunks per row
  constexpr int KCH = BN * CPR;               // K chunks per block
  constexpr int KCT = (KCH + NTH - 1) / NTH;
  constexpr int VIT = (BN / 4) * CPR;         // V items (4 keys x one chunk) per block
  constexpr int VIT_T = (VIT + NTH - 1) / NTH;

  __shared__ __align__(16) T Ks[BN * KLD];
  __shared__ __align__(16) T Vt[DP * VLD];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int li = lane & 15;
  const int lg = lane >> 4;

  // ---- which (query block, sequence, head) ----
  const int bid = blockIdx.x;
  const int h = bid % p.H;
  const int rest = bid / p.H;
  const int seq = rest % p.nseq;
  const int qb = p.nqb - 1 - rest / p.nseq;

  int TQs, TKs, qs;
  int64_t qoff, koff, voff, yoff, soff;  // element offsets of (seq, head) row 0; soff: stats row 0
  if (p.cu) {
    const int r0 = p.cu[seq];
    TQs = p.cu[seq + 1] - r0;
    TKs = TQs;
    qs = 0;
    qoff = int64_t(r0) * p.q_sr;
    koff = int64_t(r0) * p.k_sr;
    voff = int64_t(r0) * p.v_sr;
    yoff = int64_t(r0) * p.y_sr;
    soff = int64_t(h) * p.total_rows + r0;
  } else {
    TQs = p.TQ;
    TKs = p.TK;
    qs = p.q_start;
    qoff = int64_t(seq) * p.q_sb;
    koff = int64_t(seq) * p.k_sb;
    voff = int64_t(seq) * p.v_sb;
    yoff = int64_t(seq) * p.y_sb;
    soff = (int64_t(seq) * p.H + h) * p.TQ;
  }
  if (qb * BM >= TQs) return;  // uniform across the workgroup
  const T* qbase = reinterpret_cast<const T*>(p.p1) + qoff + int64_t(h) * p.q_sh;
  const T* kbase = reinterpret_cast<const T*>(p.p2) + koff + int64_t(h) * p.k_sh;
  const T* vbase = reinterpret_cast<const T*>(p.info) + voff + int64_t(h) * p.v_sh;
  T* ybase = reinterpret_cast<T*>(p.y) + yoff + int64_t(h) * p.y_sh;
  const int D = p.D;

  // ---- the wave's queries: B fragments of Q^T, loaded once ----
  const int q0 = qb * BM + wave * 32;  // local index of the wave's first query
  const bool wave_active = q0 < TQs;
  Frag qf[2][KS];
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    const int qi = q0 + 16 * s + li;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int d0 = 32 * ks + 8 * lg;
      if (qi < TQs && d0 < D) {
        qf[s][ks] = E::load8(qbase + int64_t(qi) * p.q_sr + d0);
      } else {
        qf[s][ks] = E::zero();
      }
    }
  }
  const int qlast_wg = min(TQs, (qb + 1) * BM) - 1;
  const int kend = qs + qlast_wg;  // keys j < kend are somebody's strict past
  const int nkb = (kend + BN - 1) / BN;
  const int wave_kend = wave_active ? qs + min(q0 + 32, TQs) - 1 : 0;
  const int wave_q0abs = qs + q0;
  int qabs[2];
  qabs[0] = qs + q0 + li;
  qabs[1] = qs + q0 + 16 + li;

  const float c2 = p.scale * kLog2e;
  float m_run[2] = {kNegInf, kNegInf};
  float l_run[2] = {0.f, 0.f};
  f32x4 oacc[DT][2];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int s = 0; s < 2; ++s) oacc[dt][s] = f32x4{0.f, 0.f, 0.f, 0.f};

  Chunk kreg[KCT];
  Chunk vreg[VIT_T][4];

  auto load_block = [&](int kb) {
    const int j0 = kb * BN;
#pragma unroll
    for (int c = 0; c < KCT; ++c) {
      const int idx = tid + c * NTH;
      const int row = idx / CPR, cc = idx % CPR;
      const int j = j0 + row;
      const bool ok = idx < KCH && j < TKs && cc * EPC < D;
      kreg[c] = ok ? load_chunk(kbase + int64_t(j) * p.k_sr + cc * EPC) : zero_chunk();
    }
#pragma unroll
    for (int c = 0; c < VIT_T; ++c) {
      const int it = tid + c * NTH;
      const int kq = it % (BN / 4), cc = it / (BN / 4);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int j = j0 + 4 * kq + r;
        const bool ok = it < VIT && j < TKs && cc * EPC < D;
        vreg[c][r] = ok ? load_chunk(vbase + int64_t(j) * p.v_sr + cc * EPC) : zero_chunk();
      }
    }
  };

  auto store_block = [&]() {
#pragma unroll
    for (int c = 0; c < KCT; ++c) {
      const int idx = tid + c * NTH;
      if (idx < KCH) {
        const int row = idx / CPR, cc = idx % CPR;
        store_chunk(&Ks[row * KLD + cc * EPC], kreg[c]);
      }
    }
#pragma unroll
    for (int c = 0; c < VIT_T; ++c) {
      const int it = tid + c * NTH;
      if (it < VIT) {
        const int kq = it % (BN / 4), cc = it / (BN / 4);
        if constexpr (sizeof(T) == 2) {
          // 8 head-dim rows x 4 keys: rows cc*8 + e, columns 4kq .. 4kq+3
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const int w = e >> 1, sh = (e & 1) * 16;
            const uint32_t a0 = (vreg[c][0].w[w] >> sh) & 0xffffu;
            const uint32_t a1 = (vreg[c][1].w[w] >> sh) & 0xffffu;
            const uint32_t a2 = (vreg[c][2].w[w] >> sh) & 0xffffu;
            const uint32_t a3 = (vreg[c][3].w[w] >> sh) & 0xffffu;
            uint2 v;
            v.x = a0 | (a1 << 16);
            v.y = a2 | (a3 << 16);
            *reinterpret_cast<uint2*>(&Vt[(cc * 8 + e) * VLD + 4 * kq]) = v;
          }
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            uint4 v;
            v.x = vreg[c][0].w[e];
            v.y = vreg[c][1].w[e];
            v.z = vreg[c][2].w[e];
            v.w = vreg[c][3].w[e];
            *reinterpret_cast<uint4*>(&Vt[(cc * 4 + e) * VLD + 4 * kq]) = v;
          }
        }
      }
    }
  };

  if (nkb > 0) load_block(0);
  for (int kb = 0; kb < nkb; ++kb) {
    __syncthreads();
    store_block();
    __syncthreads();
    if (kb + 1 < nkb) load_block(kb + 1);

    const int j0 = kb * BN;
    if (!wave_active || j0 >= wave_kend) continue;  // nothing in this block is in the wave's past
    const bool masked = j0 + BN > wave_q0abs;

    // S^T = K Q^T for NT key tiles x 2 query tiles
    f32x4 sacc[NT][2];
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int s = 0; s < 2; ++s) sacc[t][s] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const Frag kf = E::load8(&Ks[(16 * t + li) * KLD + 32 * ks + 8 * lg]);
#pragma unroll
        for (int s = 0; s < 2; ++s) sacc[t][s] = E::mma(kf, qf[s][ks], sacc[t][s]);
      }
    }

    // exchange scores in log2 units and the block max per query
    float bmax[2];
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      float mx = kNegInf;
#pragma unroll
      for (int t = 0; t < NT; ++t) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float u2 = sacc[t][s][r] * c2;
          float e = u2 * frcp(1.0f + fexp2(-u2));
          if (masked) {
            const int j = j0 + 16 * t + 4 * lg + r;
            if (j >= qabs[s]) e = kNegInf;
          }
          sacc[t][s][r] = e;
          mx = fmaxf(mx, e);
        }
      }
      mx = fmaxf(mx, wave_xor(mx, 16));
      mx = fmaxf(mx, wave_xor(mx, 32));
      bmax[s] = mx;
    }
    const bool need = (bmax[0] > m_run[0] + kRescale) || (bmax[1] > m_run[1] + kRescale);
    if (__ballot(need) != 0ull) {
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const float mn = bmax[s] > m_run[s] + kRescale ? bmax[s] : m_run[s];
        const float alpha = fexp2(m_run[s] - (mn == kNegInf ? 0.f : mn));
        l_run[s] *= alpha;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) oacc[dt][s] *= alpha;
        m_run[s] = mn;
      }
    }
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const float ms = m_run[s] == kNegInf ? 0.f : m_run[s];
#pragma unroll
      for (int t = 0; t < NT; ++t) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float pr = fexp2(sacc[t][s][r] - ms);
          l_run[s] += pr;
          sacc[t][s][r] = pr;
        }
      }
    }

    // O^T += V^T P^T, 32 keys per step
#pragma unroll
    for (int kk = 0; kk < NT / 2; ++kk) {
      Frag pf[2];
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        float pv[8];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          pv[r] = sacc[2 * kk][s][r];
          pv[4 + r] = sacc[2 * kk + 1][s][r];
        }
        pf[s] = E::from_f32(pv);
      }
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const T* vrow = &Vt[(16 * dt + li) * VLD + 32 * kk + 4 * lg];
        const Frag vf = E::load4x2(vrow, vrow + 16);
#pragma unroll
        for (int s = 0; s < 2; ++s) oacc[dt][s] = E::mma(vf, pf[s], oacc[dt][s]);
      }
    }
  }

  if (!wave_active) return;

  // ---- epilogue ----
  const float lam = *p.lam;
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    float lt = l_run[s];
    lt += wave_xor(lt, 16);
    lt += wave_xor(lt, 32);
    const int qi = q0 + 16 * s + li;
    const bool qv = qi < TQs;
    const int qa = qs + qi;
    const bool has = lt > 0.f;
    const float lse = has ? (m_run[s] + __log2f(lt)) * kLn2 : kNegInf;
    const float inv_l = has ? 1.0f / lt : 0.f;
    // Self score U_ii from the query's own key row
    float ud = 0.f;
    if (qv) {
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const int d0 = 32 * ks + 8 * lg;
        if (d0 < D) {
          const Frag kr = E::load8(kbase + int64_t(qa) * p.k_sr + d0);
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            float a, b;
            if constexpr (sizeof(T) == 2) {
              a = (float)qf[s][ks].v[j];
              b = (float)kr.v[j];
            } else {
              a = qf[s][ks].v[j];
              b = kr.v[j];
            }
            ud = fmaf(a, b, ud);
          }
        }
      }
    }
    ud += wave_xor(ud, 16);
    ud += wave_xor(ud, 32);
    const float sself = sigmoid_acc(ud * p.scale * p.tau_inv);
    const float gate = has ? sigmoid_acc(lse - lam * logf((float)qa + 1.0f) - sself) : 0.f;
    if (!qv) continue;
    const T* irow = vbase + int64_t(qa) * p.v_sr;
    T* yrow = ybase + int64_t(qi) * p.y_sr;
    float* brow = p.ibar + (soff + qi) * int64_t(D);
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      const int d0 = 16 * dt + 4 * lg;
      if (d0 >= D) continue;
      float ib[4], yv[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        ib[r] = oacc[dt][s][r] * inv_l;
        yv[r] = (1.0f - gate) * E::to_f(irow[d0 + r]) + gate * ib[r];
      }
      if constexpr (sizeof(T) == 2) {
        uint2 pk;
        pk.x = uint32_t(f2bf(yv[0])) | (uint32_t(f2bf(yv[1])) << 16);
        pk.y = uint32_t(f2bf(yv[2])) | (uint32_t(f2bf(yv[3])) << 16);
        *reinterpret_cast<uint2*>(yrow + d0) = pk;
      } else {
        *reinterpret_cast<float4*>(yrow + d0) = make_float4(yv[0], yv[1], yv[2], yv[3]);
      }
      *reinterpret_cast<float4*>(brow + d0) = make_float4(ib[0], ib[1], ib[2], ib[3]);
    }
    if (lg == 0) {
      p.lse[soff + qi] = lse;
      p.g[soff + qi] = gate;
    }
  }
}

// ------------------------------------------------------------------------------------------------
// bf16 tile kernel for D in {32, 64, 96, 128}
//
// One workgroup of four waves per 64 query rows of one (sequence, head). P2 and I~ blocks of 64 rows
// are staged global -> LDS (tiles.hpp), double-buffered. Wave w owns the 32 x 32 quadrant (query
// half qh = w / 2, key half kh = w % 2) of every 64 x 64 block, so each query row is covered by two
// waves with separate online-softmax states (m, l, O) that merge through LDS at the end; quadrants
// with no visible (key < query) pair are skipped. Per block and wave:
//   S^T = K Q^T       A = K rows (ds_read_b128), B = the wave's queries (registers, loaded once)
//   e   = SiLU(S^T / sqrt(D)) in log2 units, masked on the diagonal blocks
//   online softmax per query column, rescaled only when a block raises the max by more than 2^8
//   O^T += V^T P^T    A = I~ columns by ds_read_b64_tr_b16, B = P^T from the S^T accumulators
//                     (a lane holds one query and keys 4g + r of each 16-key tile: the permuted k
//                     order both fragments share)
// ------------------------------------------------------------------------------------------------
// The running reference m of a query's online softmax is an upper bound of its exponents rather
// than their maximum: with u2 = U log2e, the exponent SiLU(U) log2e = u2 sigmoid(U) never exceeds
// max(u2, 0), so the block's bound comes from the raw dot products (one max per element, no SiLU
// needed first) and m starts at 0. Exponents then stay in [-0.4, 0] below the bound for u2 >= 0
// and the row sum l is exact up to rounding whatever m is; LSE = (m + log2 l) ln2.
// The row sums come from the P^T fragments too: one more product with a fragment whose row 0 is
// all ones adds sum_k P[k][q] into row 0 of `lacc`.
// S^T = K Q^T for the wave's quadrant: keys 32 kh + 16 kt + 4 lg + r (rows), query 16 s + li.
template <int DP>
__device__ __forceinline__ void fwd_scores(const bf16_t* Ks, const typename Elem<bf16_t>::Frag (&qf)[2][DP / 32],
                                           f32x4 (&sacc)[2][2], int kh, int li, int lg) {
  using E = Elem<bf16_t>;
  using Frag = E::Frag;
  constexpr int KS = DP / 32;
#pragma unroll
  for (int kt = 0; kt < 2; ++kt)
#pragma unroll
    for (int s = 0; s < 2; ++s) sacc[kt][s] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
      const Frag kf = tile_row_frag<DP>(Ks, 32 * kh + 16 * kt + li, 4 * ks + lg);
#pragma unroll
      for (int s = 0; s < 2; ++s) sacc[kt][s] = E::mma(kf, qf[s][ks], sacc[kt][s]);
    }
  }
}

// Online softmax of one quadrant's scores and O^T += V^T P^T.
// The running reference m of a query's online softmax is an upper bound of its exponents rather
// than their maximum: with u2 = U log2e, the exponent SiLU(U) log2e = u2 sigmoid(U) never exceeds
// max(u2, 0), so the block's bound comes from the raw dot products (one max per element, no SiLU
// needed first) and m starts at 0. Exponents then stay within 0.4 below the bound for u2 >= 0, and
// the row sum l is exact up to rounding whatever m is; LSE = (m + log2 l) ln2.
// The row sums come from the P^T fragments too: one more product with a fragment whose row 0 is
// all ones adds sum_k P[k][q] into row 0 of `lacc`.
template <int DP, bool MASKED>
__device__ __forceinline__ void fwd_softmax_pv(const bf16_t* Vs, const f32x4 (&sacc)[2][2], f32x4 (&oacc)[DP / 16][2],
                                               f32x4 (&lacc)[2], float (&m_run)[2], const typename Elem<bf16_t>::Frag& ones,
                                               int key0, const int (&qabs)[2], float c2, int kh, int li, int lg) {
  using E = Elem<bf16_t>;
  using Frag = E::Frag;
  constexpr int DT = DP / 16;
  Frag vfr[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) vfr[dt] = tile_tr_frag<DP>(Vs, 32 * kh, dt, li, lg);
  __builtin_amdgcn_sched_barrier(0);
  bool keep[2][2][4];
#pragma unroll
  for (int s = 0; s < 2; ++s)
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int r = 0; r < 4; ++r) keep[s][kt][r] = !MASKED || key0 + 16 * kt + 4 * lg + r < qabs[s];
  float bnd[2];
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    float mx = kNegInf;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int r = 0; r < 4; ++r) mx = fmaxf(mx, keep[s][kt][r] ? sacc[kt][s][r] : kNegInf);
    bnd[s] = mx;
  }
  // Whether any query's bound exceeds its reference by the slack needs no reduction over the lane
  // groups: some lane's own maximum exceeds it exactly when the query's maximum does (c2 > 0 and the
  // reference is at least 0). The query's maximum is formed only in the rare rescale branch.
  const bool need = (bnd[0] * c2 > m_run[0] + kRescale) || (bnd[1] * c2 > m_run[1] + kRescale);
  if (__ballot(need) != 0ull) {
    asm volatile("" ::: "memory");  // a real branch: the rescale is rare
    lanegroup_max2(bnd[0], bnd[1]);
#pragma unroll
    for (int s = 0; s < 2; ++s) bnd[s] = fmaxf(bnd[s] * c2, 0.f);
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const float mn = bnd[s] > m_run[s] + kRescale ? bnd[s] : m_run[s];
      const float alpha = fexp2(m_run[s] - mn);
      lacc[s] *= alpha;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) oacc[dt][s] *= alpha;
      m_run[s] = mn;
    }
  }
  Frag pf[2];
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    float pv[8];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float u2 = sacc[kt][s][r] * c2;
        const float sg = frcp(1.0f + fexp2(-u2));
        const float pr = fexp2(fmaf(u2, sg, -m_run[s]));
        pv[4 * kt + r] = keep[s][kt][r] ? pr : 0.f;
      }
    pf[s] = E::from_f32(pv);
    lacc[s] = E::mma(ones, pf[s], lacc[s]);
  }
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) {
#pragma unroll
    for (int s = 0; s < 2; ++s) oacc[dt][s] = E::mma(vfr[dt], pf[s], oacc[dt][s]);
  }
}

// LDS of the tile kernels: a ring of NSTG stages (P2 tile, I~ tile); a block waits only for its own
// stage, the next NSTG - 2 stay in flight across its math (three stages: 72 KB at DP = 96, so two
// workgroups still share a CU).
template <int DP>
struct FwdTileShape {
  static constexpr int TILE = 64 * DP;
  static constexpr int STAGE = 2 * TILE;
  static constexpr int NSTG = DP <= 96 ? 3 : 2;
  static constexpr int LDS = NSTG * STAGE;
};

// One (query block, sequence, head) of the tile forward (or one key-range half of it when split),
// by its block id (the launch order: head fastest, then (when split) the halves, then query blocks
// longest first); every wave of the workgroup calls it.
template <int DP>
__device__ __forceinline__ void fwd_tile_job(const FwdParams& p, const int bid, bf16_t* smem) {
  using E = Elem<bf16_t>;
  using Frag = E::Frag;
  constexpr int KS = DP / 32, DT = DP / 16, TILE = 64 * DP;
  constexpr int STAGE = FwdTileShape<DP>::STAGE;
  constexpr int RLD = DP + 4;      // fp32 row stride of the merge buffer
  constexpr int NSTG = FwdTileShape<DP>::NSTG;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: staging in scalar registers
  const int li = lane & 15, lg = lane >> 4;
  const int kh = wave & 1, qh = wave >> 1;
  const int h = bid % p.H;
  const int half = p.part ? (bid / p.H) & 1 : 0;
  const int rest = p.part ? bid / p.H / 2 : bid / p.H;
  const int seq = rest % p.nseq;
  const int qb = p.nqb - 1 - rest / p.nseq;

  int TQs, TKs, qs;
  int64_t qoff, koff, voff, yoff, soff;
  if (p.cu) {
    const int r0 = p.cu[seq];
    TQs = p.cu[seq + 1] - r0;
    TKs = TQs;
    qs = 0;
    qoff = int64_t(r0) * p.q_sr;
    koff = int64_t(r0) * p.k_sr;
    voff = int64_t(r0) * p.v_sr;
    yoff = int64_t(r0) * p.y_sr;
    soff = int64_t(h) * p.total_rows + r0;
  } else {
    TQs = p.TQ;
    TKs = p.TK;
    qs = p.q_start;
    qoff = int64_t(seq) * p.q_sb;
    koff = int64_t(seq) * p.k_sb;
    voff = int64_t(seq) * p.v_sb;
    yoff = int64_t(seq) * p.y_sb;
    soff = (int64_t(seq) * p.H + h) * p.TQ;
  }
  if (qb * 64 >= TQs) return;
  const bf16_t* qbase = reinterpret_cast<const bf16_t*>(p.p1) + qoff + int64_t(h) * p.q_sh;
  const bf16_t* kbase = reinterpret_cast<const bf16_t*>(p.p2) + koff + int64_t(h) * p.k_sh;
  const bf16_t* vbase = reinterpret_cast<const bf16_t*>(p.info) + voff + int64_t(h) * p.v_sh;
  bf16_t* ybase = reinterpret_cast<bf16_t*>(p.y) + yoff + int64_t(h) * p.y_sh;

  const int q0 = qb * 64 + 32 * qh;  // the wave's first query row
  Frag qf[2][KS];
  int qabs[2];
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    const int qi = q0 + 16 * s + li;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
      qf[s][ks] = qi < TQs ? E::load8(qbase + int64_t(qi) * p.q_sr + 32 * ks + 8 * lg) : E::zero();
    qabs[s] = qs + qi;
  }
  const int qlast = min(TQs, qb * 64 + 64) - 1;
  const int nkb = (qs + qlast + 63) / 64;       // keys j < qs + qlast
  const int wq_last = min(q0 + 31, TQs - 1);    // the wave's last query row
  // long query blocks run as two workgroups over the two halves of their key blocks
  const bool split = p.part != nullptr && nkb > p.split_c;
  if (half == 1 && !split) return;
  const int kb_mid = split ? (nkb + 1) / 2 : nkb;
  const int kb_lo = half ? kb_mid : 0, kb_hi = half ? nkb : kb_mid;

  const bf16_t* srcs[2] = {kbase, vbase};
  const int64_t strides[2] = {p.k_sr, p.v_sr};
  TileStager<DP, 4, 2> st;
  st.init(wave, lane, strides);
  const float c2 = p.scale * kLog2e;
  float m_run[2] = {0.f, 0.f};
  f32x4 lacc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
  f32x4 oacc[DT][2];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int s = 0; s < 2; ++s) oacc[dt][s] = f32x4{0.f, 0.f, 0.f, 0.f};
  Frag ones;  // row 0 of the A operand all ones: the product sums P^T over its keys
  {
    const __bf16 one = (__bf16)(li == 0 ? 1.0f : 0.0f);
    ones.v = bf16x8{one, one, one, one, one, one, one, one};
  }

  // Block kb goes to ring slot (kb - kb_lo) % NSTG. Every step issues one block, past the end a
  // reload of the last one, so that the wait before a step always leaves the same count in flight.
  constexpr int PER = TileStager<DP, 4, 2>::PER;  // transfers per stage and wave
  auto issue_kb = [&](int kb, int slot) {
    st.issue(smem + slot * STAGE, srcs, strides, min(kb, kb_hi - 1) * 64, TKs - 1, wave, lane);
  };
  if (kb_lo < kb_hi) issue_kb(kb_lo, 0);
  __builtin_amdgcn_s_waitcnt(0);  // unconditional: no query-fragment load stays pending into the loop
  // The fragments pass through an empty asm: the compiler's own count of outstanding loads then has
  // no load of them left to wait for inside the loop (it otherwise waited for every load in flight,
  // the ring's prefetches included, before the first product of each block).
#pragma unroll
  for (int s = 0; s < 2; ++s)
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) asm volatile("" : "+v"(qf[s][ks].v));
  if (kb_lo < kb_hi && NSTG > 2) issue_kb(kb_lo + 1, 1);
  // key blocks wholly before the workgroup's first query position first (unmasked block math), then
  // the diagonal ones (masked): two loops keep one register assignment of the accumulators each
  // slotv: the block's ring slot, (kb - kb_lo) % NSTG, a constant in the unmasked loop's rounds of
  // NSTG blocks (the LDS offsets of the block's reads then fold into the read instructions)
  auto step = [&](int kb, auto masked, auto slotv) {
    const int slot = slotv;
    MOTE_STAMP(0, kb);
    __builtin_amdgcn_s_waitcnt(kVmWaitStage<(NSTG - 2) * PER>());  // this wave's part of block kb is in
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0) only (vmcnt and expcnt at their maxima)
    __builtin_amdgcn_s_barrier();  // every wave's part of block kb is in; every wave is done with block kb - 1's slot
    MOTE_STAMP(3, kb);
    issue_kb(kb + NSTG - 1, slot == 0 ? NSTG - 1 : slot - 1);
    MOTE_STAMP(1, kb);
    const bf16_t* Ks = smem + slot * STAGE;
    const int key0 = kb * 64 + 32 * kh;
    if (q0 < TQs && key0 < qs + wq_last) {
      f32x4 sacc[2][2];
      fwd_scores<DP>(Ks, qf, sacc, kh, li, lg);
      fwd_softmax_pv<DP, decltype(masked)::value>(Ks + TILE, sacc, oacc, lacc, m_run, ones, key0, qabs, c2, kh, li,
                                                  lg);
    }
    MOTE_STAMP(2, kb);
  };
  const int kb_m = min(kb_hi, (qs + qb * 64) / 64);
  int kb = kb_lo;
  for (; kb + NSTG <= kb_m; kb += NSTG)
    static_for<NSTG>([&](auto u) { step(kb + decltype(u)::value, std::false_type{}, u); });
  int slot = 0;  // (kb - kb_lo) % NSTG after whole rounds
  for (; kb < kb_m; ++kb) {
    step(kb, std::false_type{}, slot);
    slot = slot + 1 == NSTG ? 0 : slot + 1;
  }
  for (; kb < kb_hi; ++kb) {
    step(kb, std::true_type{}, slot);
    slot = slot + 1 == NSTG ? 0 : slot + 1;
  }

  // row sums: row 0 of lacc, held by lanes 0..15 (query li); broadcast to the other lane groups
  float l_run[2];
#pragma unroll
  for (int s = 0; s < 2; ++s) l_run[s] = __shfl(lacc[s][0], li, 64);
  // merge the key halves: kh = 1 hands (m, l, O) to kh = 0 through LDS
  float* R = reinterpret_cast<float*>(smem);     // [64 queries][RLD]
  float* RM = R + 64 * RLD;                      // [64] m, then [64] l
  __builtin_amdgcn_s_waitcnt(0);  // the reloads past the end have landed before the ring is reused
  __syncthreads();
  if (kh == 1) {
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const int row = 32 * qh + 16 * s + li;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) *reinterpret_cast<f32x4*>(&R[row * RLD + 16 * dt + 4 * lg]) = oacc[dt][s];
      if (lg == 0) {
        RM[row] = m_run[s];
        RM[64 + row] = l_run[s];
      }
    }
  }
  __syncthreads();
  if (kh == 1) return;
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    const int row = 32 * qh + 16 * s + li;
    const float m1 = RM[row], l1 = RM[64 + row];
    const float mm = fmaxf(m_run[s], m1);
    const float a0 = fexp2(m_run[s] - mm), a1 = fexp2(m1 - mm);
    l_run[s] = l_run[s] * a0 + l1 * a1;
    m_run[s] = mm;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
      oacc[dt][s] = oacc[dt][s] * a0 + *reinterpret_cast<const f32x4*>(&R[row * RLD + 16 * dt + 4 * lg]) * a1;
  }
  if (split) {
    // unnormalised state (O, m, l) of this half for the merge kernel
    float* part = p.part + ((((int64_t)seq * p.H + h) * p.nqb + qb) * 2 + half) * (64 * DP + 128);
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const int row = 32 * qh + 16 * s + li;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) *reinterpret_cast<f32x4*>(&part[row * DP + 16 * dt + 4 * lg]) = oacc[dt][s];
      if (lg == 0) {
        part[64 * DP + row] = m_run[s];
        part[64 * DP + 64 + row] = l_run[s];
      }
    }
    return;
  }

  const float lam = *p.lam;
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    const float lt = l_run[s];
    const int qi = q0 + 16 * s + li;
    const bool qv = qi < TQs;
    const int qa = qs + qi;
    const bool has = lt > 0.f;
    const float lse = has ? (m_run[s] + __log2f(lt)) * kLn2 : kNegInf;
    const float inv_l = has ? 1.0f / lt : 0.f;
    float ud = 0.f;
    if (qv) {
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const Frag kr = E::load8(kbase + int64_t(qa) * p.k_sr + 32 * ks + 8 * lg);
#pragma unroll
        for (int j = 0; j < 8; ++j) ud = fmaf((float)qf[s][ks].v[j], (float)kr.v[j], ud);
      }
    }
    ud += wave_xor(ud, 16);
    ud += wave_xor(ud, 32);
    const float sself = sigmoid_acc(ud * p.scale * p.tau_inv);
    const float gate = has ? sigmoid_acc(lse - lam * logf((float)qa + 1.0f) - sself) : 0.f;
    if (!qv) continue;
    const bf16_t* irow = vbase + int64_t(qa) * p.v_sr;
    bf16_t* yrow = ybase + int64_t(qi) * p.y_sr;
    float* brow = p.ibar + (soff + qi) * int64_t(DP);
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      const int d0 = 16 * dt + 4 * lg;
      const uint2 iv = *reinterpret_cast<const uint2*>(irow + d0);
      const float ivf[4] = {bf2f(iv.x & 0xffffu), bf2f(iv.x >> 16), bf2f(iv.y & 0xffffu), bf2f(iv.y >> 16)};
      float ib[4], yv[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        ib[r] = oacc[dt][s][r] * inv_l;
        yv[r] = (1.0f - gate) * ivf[r] + gate * ib[r];
      }
      uint2 pk;
      pk.x = uint32_t(f2bf(yv[0])) | (uint32_t(f2bf(yv[1])) << 16);
      pk.y = uint32_t(f2bf(yv[2])) | (uint32_t(f2bf(yv[3])) << 16);
      *reinterpret_cast<uint2*>(yrow + d0) = pk;
      *reinterpret_cast<float4*>(brow + d0) = make_float4(ib[0], ib[1], ib[2], ib[3]);
    }
    if (lg == 0) {
      p.lse[soff + qi] = lse;
      p.g[soff + qi] = gate;
    }
  }
}

template <int DP>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2)))
relation_fwd_tile_kernel(const FwdParams p) {
  __shared__ __align__(16) bf16_t smem[FwdTileShape<DP>::LDS];
  fwd_tile_job<DP>(p, blockIdx.x, smem);
}

// The same jobs taken by persistent workgroups (two per CU) from per-queue counters: queue q holds the
// heads h = q (mod jobs_nq) in launch order, and workgroup i takes from queue i % jobs_nq, so a queue's
// workgroups sit on the XCDs i % 8 = q (mod jobs_nq) (workgroups are dealt round-robin over the XCDs)
// and their L2s hold those heads' keys. With many more jobs than slots (the varlen prefill: 4,992
// workgroups of which 3,512 have rows, for 512 slots) one workgroup per job let the dispatcher stall:
// it places workgroups in order, and an XCD without a free slot holds back every later one, so 260-300
// of the 512 slots stood busy through the first half of the launch (per-workgroup stamps). The
// parameters reach each job through an opaque pointer to the kernel argument: the compiler then reads
// them (scalar loads) inside each job instead of holding every value it derives from them across the
// loop (61 scalar registers spilled, 6 now).
template <int DP>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2)))
relation_fwd_tile_persistent_kernel(const FwdParams p) {
  __shared__ __align__(16) bf16_t smem[FwdTileShape<DP>::LDS];
  __shared__ int s_job;
  const int nq = p.jobs_nq, queue = blockIdx.x % nq;
  const int hq = p.H / nq;                       // heads per queue
  const int njobs = hq * p.nseq * p.nqb;         // jobs per queue (blocks past a sequence's end included)
  for (;;) {
    if (threadIdx.x == 0)
      s_job = __hip_atomic_fetch_add(p.jobs + 32 * queue, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    const int j = __builtin_amdgcn_readfirstlane(s_job);
    if (j >= njobs) break;
    const int h = queue + nq * (j % hq), rest = j / hq;
    typedef const __attribute__((address_space(4))) FwdParams* ConstFwdParams;
    ConstFwdParams pp = (ConstFwdParams)__builtin_amdgcn_kernarg_segment_ptr();  // the kernel's one argument
    asm volatile("" : "+s"(pp));
    const FwdParams& q = *(const FwdParams*)pp;
    fwd_tile_job<DP>(q, h + q.H * rest, smem);
    __syncthreads();  // the next job reuses the LDS and s_job
  }
}

__global__ void __launch_bounds__(64) fwd_jobs_clear_kernel(int* jobs) {
  if (threadIdx.x < 8) jobs[32 * threadIdx.x] = 0;
}

// Merge of the two halves of a split query block, then the epilogue of relation_fwd_tile_kernel:
// four threads per row, each owning DP / 4 head-dim elements.
template <int DP>
__global__ void __launch_bounds__(256) relation_fwd_merge_kernel(const FwdParams p) {
  constexpr int PER = DP / 4;  // elements per thread
  const int tid = threadIdx.x;
  const int row = tid >> 2, quarter = tid & 3;
  const int bid = blockIdx.x;
  const int h = bid % p.H;
  const int rest = bid / p.H;
  const int seq = rest % p.nseq;
  const int qb = rest / p.nseq;

  int TQs, qs;
  int64_t qoff, koff, voff, yoff, soff;
  if (p.cu) {
    const int r0 = p.cu[seq];
    TQs = p.cu[seq + 1] - r0;
    qs = 0;
    qoff = int64_t(r0) * p.q_sr;
    koff = int64_t(r0) * p.k_sr;
    voff = int64_t(r0) * p.v_sr;
    yoff = int64_t(r0) * p.y_sr;
    soff = int64_t(h) * p.total_rows + r0;
  } else {
    TQs = p.TQ;
    qs = p.q_start;
    qoff = int64_t(seq) * p.q_sb;
    koff = int64_t(seq) * p.k_sb;
    voff = int64_t(seq) * p.v_sb;
    yoff = int64_t(seq) * p.y_sb;
    soff = (int64_t(seq) * p.H + h) * p.TQ;
  }
  if (qb * 64 >= TQs) return;
  const int qlast = min(TQs, qb * 64 + 64) - 1;
  const int nkb = (qs + qlast + 63) / 64;
  if (!(nkb > p.split_c)) return;  // this query block ran whole
  const float* P0 = p.part + (((int64_t)seq * p.H + h) * p.nqb + qb) * 2 * (64 * DP + 128);
  const float* P1 = P0 + (64 * DP + 128);
  const int qi = qb * 64 + row;
  const bool qv = qi < TQs;
  const int qa = qs + qi;
  const float m0 = P0[64 * DP + row], l0 = P0[64 * DP + 64 + row];
  const float m1 = P1[64 * DP + row], l1 = P1[64 * DP + 64 + row];
  const float mm = fmaxf(m0, m1);
  const float a0 = fexp2(m0 - mm), a1 = fexp2(m1 - mm);
  const float lt = l0 * a0 + l1 * a1;
  const bool has = lt > 0.f;
  const float lse = has ? (mm + __log2f(lt)) * kLn2 : kNegInf;
  const float inv_l = has ? 1.0f / lt : 0.f;
  const int d0 = quarter * PER;
  const bf16_t* qrow = reinterpret_cast<const bf16_t*>(p.p1) + qoff + int64_t(h) * p.q_sh + int64_t(qv ? qi : 0) * p.q_sr;
  const bf16_t* krow = reinterpret_cast<const bf16_t*>(p.p2) + koff + int64_t(h) * p.k_sh + int64_t(qv ? qa : 0) * p.k_sr;
  float ud = 0.f;
  if (qv) {
#pragma unroll
    for (int c = 0; c < PER; c += 8) {
      const bf16x8 q8 = *reinterpret_cast<const bf16x8*>(qrow + d0 + c);
      const bf16x8 k8 = *reinterpret_cast<const bf16x8*>(krow + d0 + c);
#pragma unroll
      for (int e = 0; e < 8; ++e) ud = fmaf((float)q8[e], (float)k8[e], ud);
    }
  }
  ud += wave_xor(ud, 1);
  ud += wave_xor(ud, 2);
  const float sself = sigmoid_acc(ud * p.scale * p.tau_inv);
  const float gate = has ? sigmoid_acc(lse - *p.lam * logf((float)qa + 1.0f) - sself) : 0.f;
  if (!qv) return;
  const bf16_t* irow = reinterpret_cast<const bf16_t*>(p.info) + voff + int64_t(h) * p.v_sh + int64_t(qa) * p.v_sr;
  bf16_t* yrow = reinterpret_cast<bf16_t*>(p.y) + yoff + int64_t(h) * p.y_sh + int64_t(qi) * p.y_sr;
  float* brow = p.ibar + (soff + qi) * int64_t(DP);
#pragma unroll
  for (int c = 0; c < PER; c += 8) {
    const bf16x8 i8 = *reinterpret_cast<const bf16x8*>(irow + d0 + c);
    float ib[8], yv[8];
#pragma unroll
    for (int e = 0; e < 8; e += 4) {
      const float4 o0 = *reinterpret_cast<const float4*>(&P0[row * DP + d0 + c + e]);
      const float4 o1 = *reinterpret_cast<const float4*>(&P1[row * DP + d0 + c + e]);
      ib[e] = (o0.x * a0 + o1.x * a1) * inv_l;
      ib[e + 1] = (o0.y * a0 + o1.y * a1) * inv_l;
      ib[e + 2] = (o0.z * a0 + o1.z * a1) * inv_l;
      ib[e + 3] = (o0.w * a0 + o1.w * a1) * inv_l;
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) yv[e] = (1.0f - gate) * (float)i8[e] + gate * ib[e];
    *reinterpret_cast<bf16x8*>(yrow + d0 + c) = Elem<bf16_t>::from_f32(yv).v;
    *reinterpret_cast<float4*>(brow + d0 + c) = make_float4(ib[0], ib[1], ib[2], ib[3]);
    *reinterpret_cast<float4*>(brow + d0 + c + 4) = make_float4(ib[4], ib[5], ib[6], ib[7]);
  }
  if (quarter == 0) {
    p.lse[soff + qi] = lse;
    p.g[soff + qi] = gate;
  }
}

// ------------------------------------------------------------------------------------------------
// host launcher
// ------------------------------------------------------------------------------------------------
template <typename T, int DP, int BN, int NW>
static void launch_fwd_t(const FwdParams& fp, int nblocks, hipStream_t stream) {
  hipLaunchKernelGGL((relation_fwd_kernel<T, DP, BN, NW>), dim3(nblocks), dim3(NW * 64), 0, stream, fp);
}

template <typename T, int BN, int NW>
static void launch_fwd_dp(const FwdParams& fp, int DP, int nblocks, hipStream_t stream) {
  switch (DP) {
    case 32: launch_fwd_t<T, 32, BN, NW>(fp, nblocks, stream); break;
    case 64: launch_fwd_t<T, 64, BN, NW>(fp, nblocks, stream); break;
    case 96: launch_fwd_t<T, 96, BN, NW>(fp, nblocks, stream); break;
    default: launch_fwd_t<T, 128, BN, NW>(fp, nblocks, stream); break;
  }
}

static bool view_ok(const mote_view& v) { return v.data != nullptr; }

// The tile kernel serves bf16 with D in {32, 64, 96, 128} and row strides below 2^24.
static bool fwd_tiles(const mote_relation_fwd_args* a) {
  return a->dtype == MOTE_BF16 && padded_dim(a->D) == a->D && tile_strides_ok(a->p1, a->p2, a->info);
}

// Key blocks of the longest query block; query blocks with more than split_c of them run as halves.
static int fwd_max_key_blocks(const mote_relation_fwd_args* a) {
  const int qs = a->cu_seqlens ? 0 : a->q_start;
  return (qs + a->TQ - 1 + 63) / 64;
}
// Measured at the Mote-96M shape (78 key blocks), splitting does not pay for the merge launch; rows
// beyond 96 key blocks (6144 positions) split.
static int fwd_split_c(const mote_relation_fwd_args* a) {
  const int n = fwd_max_key_blocks(a);
  return n > 96 ? (n + 1) / 2 : 1 << 30;
}

int device_cu_count();

// Persistent workgroups for the tile forward (one job counter per queue in the workspace) when there
// are at least four jobs per workgroup slot, as in the varlen prefill (C5: 4,992 jobs on 512 slots,
// 390 -> 331 us per layer in kernel traces; per-job stamps: 490-512 workgroups busy through the
// launch against 264-304 for its first half, though each key block then takes 1.42 against 1.25 us);
// with fewer the one-job-per-workgroup launch measured as fast or faster (C3, 624 jobs: 85.1 against
// 88.6 us). MOTE_FWD_PERSIST = 0 / 1 overrides.
static bool fwd_persistent(const mote_relation_fwd_args* a) {
  const char* e = getenv("MOTE_FWD_PERSIST");
  if (e && e[0] == '0') return false;
  if (e && e[0] == '1') return true;
  const int64_t jobs = int64_t(a->B) * a->H * ((a->TQ + 63) / 64);
  return jobs >= 4 * 2 * int64_t(device_cu_count());
}
constexpr size_t kFwdJobBytes = 8 * 32 * sizeof(int);  // eight queue counters, 128 bytes apart

size_t fwd_workspace_bytes(const mote_relation_fwd_args* a) {
  if (!a || a->TQ <= 0 || a->D <= 0 || a->D > 128 || !fwd_tiles(a)) return 0;
  if (fwd_split_c(a) >= (1 << 30)) return fwd_persistent(a) ? kFwdJobBytes : 0;
  const size_t nqb = (size_t(a->TQ) + 63) / 64;
  return size_t(a->B) * a->H * nqb * 2 * (64 * size_t(a->D) + 128) * sizeof(float);
}

int launch_fwd(const mote_relation_fwd_args* a, hipStream_t stream) {
  if (!a) return set_error(MOTE_ERR_ARGUMENT, "relation_fwd: null args");
  if (a->dtype != MOTE_F32 && a->dtype != MOTE_BF16) return set_error(MOTE_ERR_ARGUMENT, "relation_fwd: bad dtype %d", a->dtype);
  if (a->D <= 0 || a->D > 128 || a->D % 8 != 0)
    return set_error(MOTE_ERR_SHAPE, "relation_fwd: head dim %d unsupported (need 8 <= D <= 128, D %% 8 == 0)", a->D);
  if (a->B <= 0 || a->H <= 0 || a->TQ < 0) return set_error(MOTE_ERR_SHAPE, "relation_fwd: bad sizes B=%d H=%d TQ=%d", a->B, a->H, a->TQ);
  if (a->cu_seqlens) {
    if (a->q_start != 0) return set_error(MOTE_ERR_SHAPE, "relation_fwd: varlen mode needs q_start == 0");
    if (a->TK != a->TQ) return set_error(MOTE_ERR_SHAPE, "relation_fwd: varlen mode needs TK == TQ (the longest sequence)");
  } else if (a->TK != a->q_start + a->TQ) {
    return set_error(MOTE_ERR_SHAPE, "relation_fwd: keys must cover the cached prefix plus the new rows (TK=%d, q_start=%d, TQ=%d)",
                     a->TK, a->q_start, a->TQ);
  }
  if (a->TQ == 0) return MOTE_OK;  // empty outputs: nothing to launch (their pointers may be null)
  if (!view_ok(a->p1) || !view_ok(a->p2) || !view_ok(a->info) || !view_ok(a->y) || !a->ibar || !a->lse || !a->g || !a->lam)
    return set_error(MOTE_ERR_ARGUMENT, "relation_fwd: null tensor pointer");
  FwdParams fp{};
  fp.p1 = a->p1.data;
  fp.p2 = a->p2.data;
  fp.info = a->info.data;
  fp.y = a->y.data;
  fp.ibar = a->ibar;
  fp.lse = a->lse;
  fp.g = a->g;
  fp.lam = a->lam;
  fp.cu = a->cu_seqlens;
  fp.q_sb = a->p1.stride_b; fp.q_sh = a->p1.stride_h; fp.q_sr = a->p1.stride_r;
  fp.k_sb = a->p2.stride_b; fp.k_sh = a->p2.stride_h; fp.k_sr = a->p2.stride_r;
  fp.v_sb = a->info.stride_b; fp.v_sh = a->info.stride_h; fp.v_sr = a->info.stride_r;
  fp.y_sb = a->y.stride_b; fp.y_sh = a->y.stride_h; fp.y_sr = a->y.stride_r;
  fp.nseq = a->B;
  fp.H = a->H;
  fp.TQ = a->TQ;
  fp.TK = a->TK;
  fp.D = a->D;
  fp.q_start = a->q_start;
  fp.total_rows = a->total_rows;
  fp.scale = 1.0f / sqrtf((float)a->D);
  fp.tau_inv = 1.0f / a->tau_s;
  const int DP = padded_dim(a->D);
  // Four waves (128 query rows) per workgroup when that still gives two workgroups per CU;
  // otherwise two waves (64 rows) to spread short problems over more CUs.
  const int64_t units = int64_t(a->B) * a->H;
  const int nqb4 = (a->TQ + 127) / 128;
  const bool wide = units * nqb4 >= 512;
  if (fwd_tiles(a)) {
    fp.nqb = (a->TQ + 63) / 64;
    const size_t need = fwd_workspace_bytes(a);
    const bool have = need > 0 && a->workspace && a->workspace_bytes >= need;
    const bool split = have && fwd_split_c(a) < (1 << 30);
    const bool persist = have && !split;  // (the workspace then holds the job counters)
    fp.part = split ? reinterpret_cast<float*>(a->workspace) : nullptr;
    fp.split_c = split ? fwd_split_c(a) : (1 << 30);
    fp.jobs = persist ? reinterpret_cast<int*>(a->workspace) : nullptr;
    fp.jobs_nq = a->H % 8 == 0 ? 8 : a->H % 4 == 0 ? 4 : a->H % 2 == 0 ? 2 : 1;
    const int nb = int(units * fp.nqb);
    const int resident = 2 * device_cu_count();
    const int pgrid = (resident < nb ? resident : nb) / fp.jobs_nq * fp.jobs_nq;
    if (persist) hipLaunchKernelGGL(fwd_jobs_clear_kernel, dim3(1), dim3(64), 0, stream, fp.jobs);
#define MOTE_FWD_TILE(DPV)                                                                                      \
  if (persist) {                                                                                                \
    hipLaunchKernelGGL((relation_fwd_tile_persistent_kernel<DPV>), dim3(pgrid > 0 ? pgrid : fp.jobs_nq), dim3(256), 0, \
                       stream, fp);                                                                             \
  } else {                                                                                                      \
    hipLaunchKernelGGL((relation_fwd_tile_kernel<DPV>), dim3(split ? 2 * nb : nb), dim3(256), 0, stream, fp);    \
    if (split) hipLaunchKernelGGL((relation_fwd_merge_kernel<DPV>), dim3(nb), dim3(256), 0, stream, fp);          \
  }
    switch (DP) {
      case 32: MOTE_FWD_TILE(32) break;
      case 64: MOTE_FWD_TILE(64) break;
      case 96: MOTE_FWD_TILE(96) break;
      default: MOTE_FWD_TILE(128) break;
    }
#undef MOTE_FWD_TILE
  } else if (a->dtype == MOTE_BF16) {
    if (wide) {
      fp.nqb = nqb4;
      launch_fwd_dp<bf16_t, 64, 4>(fp, DP, int(units * fp.nqb), stream);
    } else {
      fp.nqb = (a->TQ + 63) / 64;
      launch_fwd_dp<bf16_t, 64, 2>(fp, DP, int(units * fp.nqb), stream);
    }
  } else {
    if (wide) {
      fp.nqb = nqb4;
      launch_fwd_dp<float, 32, 4>(fp, DP, int(units * fp.nqb), stream);
    } else {
      fp.nqb = (a->TQ + 63) / 64;
      launch_fwd_dp<float, 32, 2>(fp, DP, int(units * fp.nqb), stream);
    }
  }
  return check_launch("relation_fwd");
}

}  // namespace mote
