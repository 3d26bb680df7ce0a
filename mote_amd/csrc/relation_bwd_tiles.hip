// Atomic-free Relation backward for bf16, D in {32, 64, 96, 128} (mote/model/flash_relation.py:10-15
// for the algebra; the reference's two-pass `_bwd_kv_kernel` / `_bwd_q_kernel`, :370-460, has the
// same split of the work).
//
// Both kernels walk 64 x 64 blocks of the (query, key) plane; a wave owns a 32 x 32 quadrant (query
// half qh, key half kh) of every block of its workgroup, so a block costs a quarter of the latency it
// would on one wave and fully masked quadrants of the diagonal blocks are skipped. Operand tiles of
// 64 rows are staged global -> LDS with global_load_lds (tiles.hpp).
//
// Per element (query i, key j < i) with U = <P1_i, P2_j> / sqrt(D), sg = sigmoid(U), L = LSE_i:
//   w = exp(SiLU(U) - L)  (computed as exp2(U log2e sg - L log2e)),
//   dE = w (dW + c_i) with dW = <dI-bar_i, I~_j> and c_i = dA_i - Delta_i,
//   dU = dE SiLU'(U),     SiLU'(U) = sg + U sg (1 - sg).
//
// Key kernel (one workgroup per 64 keys of one (batch, head), longest first): per query block
// U = Q K^T and dW = dI-bar V^T with queries in the accumulator rows and the wave's keys in the
// columns, so w and dU feed dV += W^T dI-bar and dK += dU^T Q as permuted-k A operands; the B
// operands (dI-bar and Q with queries along k) are ds_read_b64_tr_b16 reads of the same tiles.
// dV, dK stay in registers across query blocks; the two query-half waves of a key half add through
// LDS at the end, then the Self terms of keys that are also queries ((1 - g) dY into dI~ and
// dU_ii P1 into dP2) and 16-byte stores.
//
// The key kernel also stores dU, for every visible (query block, key block) pair, in the register
// layout its waves hold it in (keys in lanes). Query kernel (one workgroup of eight waves per two
// query blocks, longest first): per key block, dQ^T += K^T dU^T with both operands from transposed
// LDS reads, of the staged P2 tile and of the staged dU fragments; no elementwise work and no
// recomputed products. The
// key-half waves add through LDS; the Self part dU_ii P2_i joins before the store.
#include <type_traits>
#include <utility>

#include "common.hpp"
#include "bwd.hpp"
#include "tiles.hpp"

namespace mote {

__device__ __forceinline__ int lane_of(int li, int lg) { return 16 * lg + li; }

// dU of the wave's quadrant for the dQ kernel, stored as the wave holds it: au[kt] has key 16 kt + li
// and, in slots 4 qt + r, query 16 qt + 4 lg + r. Lane L writes au[kt] whole, one 16-byte chunk per
// key tile at position dut_pos(L) of the tile's 1 KB region. The dQ kernel reads the transpose
// (queries in lanes) with ds_read_b64_tr_b16 (dut_frag); dut_pos spreads the sixteen 8-byte pieces
// of one transposed read over the banks.
__device__ __forceinline__ int dut_pos(int L) { return L ^ (((L >> 4) & 3) << 2); }

__device__ __forceinline__ void store_dut(const Elem<bf16_t>::Frag (&au)[2], bf16_t* dst, int lane) {
  const int off = dut_pos(lane) * 8;
  *reinterpret_cast<bf16x8*>(dst + off) = au[0].v;
  *reinterpret_cast<bf16x8*>(dst + 512 + off) = au[1].v;
}

// The dQ product's B fragment of query tile qt from the 2 KB that one key-kernel wave stored (staged
// in LDS at `reg`): lane (li = 4 k + m, lg) points at key 4 lg + k of each key tile, queries
// 16 qt + 4 m .. + 3, and receives query 16 qt + li of keys 4 lg .. 4 lg + 3 (slots 0..3, key tile 0)
// and 16 + 4 lg .. + 3 (slots 4..7, key tile 1): the k order of tile_tr_frag.
__device__ __forceinline__ Elem<bf16_t>::Frag dut_frag(const bf16_t* reg, int qt, int li, int lg) {
  const int k = li >> 2, m = li & 3;
  const bf16_t* p = reg + dut_pos(16 * m + 4 * lg + k) * 8 + qt * 4;
  const bf16x4 lo = lds_tr4(p), hi = lds_tr4(p + 512);
  Elem<bf16_t>::Frag f;
  f.v = bf16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  return f;
}

__device__ __forceinline__ void store_dut_zero(bf16_t* dst, int lane) {
#pragma unroll
  for (int kt = 0; kt < 2; ++kt) *reinterpret_cast<bf16x8*>(dst + kt * 512 + lane * 8) = bf16x8{};
}

// ------------------------------------------------------------------------------------------------
// key-stationary kernel: dP2 and dI~
// ------------------------------------------------------------------------------------------------
template <int DP, bool MASKED>
__device__ __forceinline__ void kv_block(const bf16_t* Qs, const bf16_t* Ds, const float* Ss, const bf16_t* Ks,
                                         const bf16_t* Vs, f32x4 (&dvacc)[2][DP / 16], f32x4 (&dkacc)[2][DP / 16],
                                         bf16_t* dut_w, int qh, int kh, int li, int lg, int key0, int qa0,
                                         float nc2) {
  using E = Elem<bf16_t>;
  using Frag = E::Frag;
  constexpr int KS = DP / 32, DT = DP / 16;
  // the query rows' statistics: lse2 (LSE in log2 units) and c = dA - Delta, which seeds the dW
  // accumulator so the product yields dW + c with no add per element
  float lv[8];
  f32x4 c4[2];
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) {
    const float4 l4 = *reinterpret_cast<const float4*>(Ss + 32 * qh + 16 * qt + 4 * lg);
    const float4 cq = *reinterpret_cast<const float4*>(Ss + 64 + 32 * qh + 16 * qt + 4 * lg);
    lv[4 * qt] = l4.x; lv[4 * qt + 1] = l4.y; lv[4 * qt + 2] = l4.z; lv[4 * qt + 3] = l4.w;
    c4[qt] = f32x4{cq.x, cq.y, cq.z, cq.w};
  }
  f32x4 sacc[2][2], wacc[2][2];  // [query tile][key tile]
#pragma unroll
  for (int qt = 0; qt < 2; ++qt)
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
      sacc[qt][kt] = f32x4{0.f, 0.f, 0.f, 0.f};
      wacc[qt][kt] = c4[qt];
    }
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    Frag kf[2], vf[2];  // the wave's keys as B fragments (k = head dim, column = key)
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
      kf[kt] = tile_row_frag<DP>(Ks, 32 * kh + 16 * kt + li, 4 * ks + lg);
      vf[kt] = tile_row_frag<DP>(Vs, 32 * kh + 16 * kt + li, 4 * ks + lg);
    }
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
      const int row = 32 * qh + 16 * qt + li;
      const Frag aq = tile_row_frag<DP>(Qs, row, 4 * ks + lg);
      const Frag ad = tile_row_frag<DP>(Ds, row, 4 * ks + lg);
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
        sacc[qt][kt] = E::mma(aq, kf[kt], sacc[qt][kt]);
        wacc[qt][kt] = E::mma(ad, vf[kt], wacc[qt][kt]);
      }
    }
  }
  // rows 32 qh + 16 qt + 4 lg + r; key 16 kt + li of the wave's half. The elementwise chain runs
  // phase by phase over the 8 elements of one key tile (two query tiles), so each transcendental's
  // result is consumed 8 instructions later instead of by the next one.
  Frag aw[2], au[2];
  float wv[2][8], uv[2][8];
#pragma unroll
  for (int kt = 0; kt < 2; ++kt) {
    float t[8], sg[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) t[e] = sacc[e >> 2][kt][e & 3] * nc2;  // -U log2e
#pragma unroll
    for (int e = 0; e < 8; ++e) sg[e] = fexp2(t[e]);
#pragma unroll
    for (int e = 0; e < 8; ++e) sg[e] = frcp(1.0f + sg[e]);             // sigmoid(U)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float w = fexp2(-fmaf(t[e], sg[e], lv[e]));                       // exp2(U log2e sg - lse2)
      if constexpr (MASKED) w = key0 + 16 * kt + li < qa0 + 16 * (e >> 2) + 4 * lg + (e & 3) ? w : 0.f;
      wv[kt][e] = w;
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      // SiLU'(U) = sg (1 + U (1 - sg)) with U (1 - sg) ln2-scaled from t: a = t (sg - 1) = U log2e (1 - sg)
      const float a = fmaf(t[e], sg[e], -t[e]);
      const float sp = sg[e] * fmaf(a, kLn2, 1.0f);
      uv[kt][e] = wv[kt][e] * wacc[e >> 2][kt][e & 3] * sp;  // wacc = dW + c
    }
    // dV += W^T dI-bar, dK += dU^T Q of key tile kt over the wave's 32 queries (k in permuted
    // order), right after kt's elementwise: tile 0's products then run beside tile 1's exponentials
    // (measured at C3: key kernel 133 -> 129.5 us, against the products of both tiles after both)
    aw[kt] = E::from_f32(wv[kt]);
    au[kt] = E::from_f32(uv[kt]);
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      const Frag bd = tile_tr_frag<DP>(Ds, 32 * qh, dt, li, lg);
      const Frag bq = tile_tr_frag<DP>(Qs, 32 * qh, dt, li, lg);
      dvacc[kt][dt] = E::mma(aw[kt], bd, dvacc[kt][dt]);
      dkacc[kt][dt] = E::mma(au[kt], bq, dkacc[kt][dt]);
    }
  }
  // both key tiles' dU in two 16-byte stores per lane (two 8-byte stores per key tile, made as each
  // tile finishes, ran the key kernel 20 % slower; the transpose into the dQ product's B layout by
  // identity products here ran the key kernel 2 % slower than the transposed reads in the dQ kernel)
  if (dut_w) store_dut(au, dut_w, lane_of(li, lg));
}

template <int DP>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(DP <= 96 ? 2 : 1)))
bwd_kv_kernel(const BwdParams p) {
  using E = Elem<bf16_t>;
  using Frag = E::Frag;
  constexpr int KS = DP / 32, DT = DP / 16, CPR = DP / 8, TILE = 64 * DP;
  constexpr int STAGE = 2 * TILE + 256;  // bf16 slots per stage: Q tile, dI-bar tile, 128 fp32 stats
  __shared__ __align__(16) bf16_t smem[2 * STAGE];
  __shared__ __align__(16) bf16_t kvs[2 * TILE];  // the workgroup's 64 P2 rows, then its 64 I~ rows

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: staging in scalar registers
  const int li = lane & 15, lg = lane >> 4;
  const int kh = wave & 1, qh = wave >> 1;
  const int BH = p.B * p.H;
  const int bh = blockIdx.x % BH;
  const int kb = blockIdx.x / BH;  // key block 0 sees the most queries: longest first
  const int b = bh / p.H, h = bh % p.H;
  const int k0 = kb * 64;
  const int nqb = p.TQp / 64;
  const bf16_t* qbase = reinterpret_cast<const bf16_t*>(p.p1) + b * p.q_sb + h * p.q_sh;
  const bf16_t* kbase = reinterpret_cast<const bf16_t*>(p.p2) + b * p.k_sb + h * p.k_sh;
  const bf16_t* vbase = reinterpret_cast<const bf16_t*>(p.info) + b * p.v_sb + h * p.v_sh;
  const bf16_t* dbase = reinterpret_cast<const bf16_t*>(p.wdib) + int64_t(bh) * p.TQp * DP;
  const float* sbase = p.stat + int64_t(bh) * nqb * 128;

  const int key0 = k0 + 32 * kh;
  f32x4 dvacc[2][DT], dkacc[2][DT];
#pragma unroll
  for (int kt = 0; kt < 2; ++kt)
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      dvacc[kt][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
      dkacc[kt][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
    }

  const bf16_t* srcs[2] = {qbase, dbase};
  const int64_t strides[2] = {p.q_sr, DP};
  TileStager<DP, 4, 2> st;
  st.init(wave, lane, strides);
  auto issue = [&](int qb, int stage) {
    bf16_t* dst = smem + stage * STAGE;
    st.issue(dst, srcs, strides, qb * 64, p.TQ - 1, wave, lane);
    if (wave == 3 && lane < 32) {
      lds_dma16_s(sbase + int64_t(qb) * 128, 16u * lane, dst + 2 * TILE);
    }
  };

  const float nc2 = -p.scale * kLog2e;
  const int qb_lo = max(0, k0 + 1 - p.q_start) / 64;
  // PairTable::offset(qb) for the block in hand, advanced by qb + A per block (offset(qb + 1) - offset(qb))
  const int pair_a = (p.q_start + 126) / 64;
  int64_t pair_off = PairTable::offset(qb_lo, p.q_start);
  // dU of this key block: pair (qb, kb) at PairTable::offset(qb) + kb, 8 KB per pair; wave (kh, qh)
  // writes its 2 KB at (kh * 4 + 2 qh) * 512 elements (store_dut)
  bf16_t* dut_bh = reinterpret_cast<bf16_t*>(p.dut) + int64_t(bh) * p.npairs * 4096 + (kh * 4 + 2 * qh) * 512;
  {
    // the key rows once (rows past the keys: finite copies whose results are never stored)
    const bf16_t* ksrc[2] = {kbase, vbase};
    const int64_t kstr[2] = {p.k_sr, p.v_sr};
    TileStager<DP, 4, 2> kst;
    kst.init(wave, lane, kstr);
    kst.issue(kvs, ksrc, kstr, k0, p.TK - 1, wave, lane);
  }
  if (qb_lo < nqb) issue(qb_lo, 0);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  // Diagonal query blocks (some key not before some query) first, with the masked block math, then
  // the rest with the unmasked math: two loops instead of a branch keeps one register assignment
  // of the accumulators per loop.
  auto step = [&](int qb, auto masked) {
    MOTE_STAMP(0, qb - qb_lo);
    const int stage = (qb - qb_lo) & 1;
    if (qb + 1 < nqb) issue(qb + 1, stage ^ 1);
    MOTE_STAMP(1, qb - qb_lo);
    const bf16_t* Qs = smem + stage * STAGE;
    const bf16_t* Ds = Qs + TILE;
    const float* Ss = reinterpret_cast<const float*>(Qs + 2 * TILE);
    const int i0 = qb * 64 + 32 * qh;   // the wave's first query row
    const int qa0 = p.q_start + i0;     // its position
    bf16_t* dut_w = kb < PairTable::nkb(qb, p.TQ, p.q_start) ? dut_bh + (pair_off + kb) * 4096 : nullptr;
    pair_off += qb + pair_a;  // PairTable::offset(qb + 1)
    // quadrant visible at all (some key < some query position), and not wholly padding rows
    if (i0 < p.TQ && key0 < qa0 + 31)
      kv_block<DP, decltype(masked)::value>(Qs, Ds, Ss, kvs, kvs + TILE, dvacc, dkacc, dut_w, qh, kh, li, lg,
                                            key0, qa0, nc2);
    else if (dut_w)
      store_dut_zero(dut_w, lane);
    MOTE_STAMP(2, qb - qb_lo);
    // The next block's transfers were issued before this block's two dU^T stores, and vector-memory
    // operations retire in issue order: waiting until at most the two stores are outstanding means the
    // transfers have landed, while the stores stay in flight across the barrier.
    if (dut_w)
      __builtin_amdgcn_s_waitcnt(kVmWaitStage<2>());
    else
      __builtin_amdgcn_s_waitcnt(kVmWaitStage<0>());
    MOTE_STAMP(3, qb - qb_lo);
    lds_barrier();
    MOTE_STAMP(4, qb - qb_lo);
  };
  // unmasked for every wave once the block's first query position exceeds the last key
  const int qb_m = min(nqb, max(qb_lo, k0 + 63 - p.q_start >= 0 ? (k0 + 63 - p.q_start) / 64 + 1 : 0));
  int qb = qb_lo;
  for (; qb < qb_m; ++qb) step(qb, std::true_type{});
  for (; qb < nqb; ++qb) step(qb, std::false_type{});

  // add the two query halves through LDS: R[0] = dV, R[1] = dK, [64 keys][DP] fp32
  float* R = reinterpret_cast<float*>(smem);
  __syncthreads();
  if (qh == 1) {
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = 32 * kh + 16 * kt + 4 * lg + r, col = 16 * dt + li;
          R[row * DP + col] = dvacc[kt][dt][r];
          R[64 * DP + row * DP + col] = dkacc[kt][dt][r];
        }
  }
  __syncthreads();
  if (qh == 0) {
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = 32 * kh + 16 * kt + 4 * lg + r, col = 16 * dt + li;
          R[row * DP + col] += dvacc[kt][dt][r];
          R[64 * DP + row * DP + col] += dkacc[kt][dt][r];
        }
  }
  __syncthreads();
  // Self terms and 16-byte stores: one chunk of 8 head-dim elements of one key row per item
  const bf16_t* dybase = reinterpret_cast<const bf16_t*>(p.dy) + b * p.y_sb + h * p.y_sh;
  bf16_t* dkout = reinterpret_cast<bf16_t*>(p.dp2) + b * p.dk_sb + h * p.dk_sh;
  bf16_t* dvout = reinterpret_cast<bf16_t*>(p.dinfo) + b * p.dv_sb + h * p.dv_sh;
  for (int item = tid; item < 64 * CPR; item += 256) {
    const int row = item / CPR, d0 = (item % CPR) * 8;
    const int j = k0 + row;
    if (j >= p.TK) continue;
    float dv[8], dk[8];
#pragma unroll
    for (int e = 0; e < 8; e += 4) {
      const float4 a = *reinterpret_cast<const float4*>(&R[row * DP + d0 + e]);
      const float4 c = *reinterpret_cast<const float4*>(&R[64 * DP + row * DP + d0 + e]);
      dv[e] = a.x; dv[e + 1] = a.y; dv[e + 2] = a.z; dv[e + 3] = a.w;
      dk[e] = c.x; dk[e + 1] = c.y; dk[e + 2] = c.z; dk[e + 3] = c.w;
    }
    const int i = j - p.q_start;
    if (i >= 0) {
      const float gs = p.g[int64_t(bh) * p.TQ + i];
      const float us = p.duii[int64_t(bh) * p.TQp + i];
      const Frag y8 = E::load8(dybase + int64_t(i) * p.y_sr + d0);
      const Frag q8 = E::load8(qbase + int64_t(i) * p.q_sr + d0);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        dv[e] = fmaf(1.0f - gs, (float)y8.v[e], dv[e]);
        dk[e] = fmaf(us, (float)q8.v[e], dk[e]);
      }
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) dk[e] *= p.scale;
    Frag ov = E::from_f32(dv), ok = E::from_f32(dk);
    *reinterpret_cast<bf16x8*>(dvout + int64_t(j) * p.dv_sr + d0) = ov.v;
    *reinterpret_cast<bf16x8*>(dkout + int64_t(j) * p.dk_sr + d0) = ok.v;
  }
}

// ------------------------------------------------------------------------------------------------
// query-stationary kernel: dP1 = (dU P2 + dU_ii P2_i) / sqrt(D) from the stored dU fragments
// ------------------------------------------------------------------------------------------------
// dQ^T of two query blocks of one (batch, head) per workgroup of eight waves: wave w takes key half kh = w % 2 and the
// 32 queries qq = w / 2 of the pair (qq / 2 = 0: the later block, 1: the earlier one). Per key block:
// A = K^T by transposed LDS reads of the staged P2 tile, B = dU^T by transposed LDS reads of the 2 KB
// the key kernel's wave (kh, qh) stored for the wave's query block (through the same ring slot). Both query blocks read one
// staged P2 tile: staging it is the kernel's largest cost (the L2 -> LDS path, shared by the CU),
// and 128 queries per workgroup stage it half as often as 64. No elementwise work: NS key blocks in
// flight (P2 tiles and fragments in an NS-deep LDS ring; the loop is unrolled by NS so every slot
// index is a constant). Query blocks pair from the top (the two longest together, longest pairs
// first); the earlier block of a pair sees at most one key block fewer, and with an odd count the
// lowest pair has one block. The key halves add through LDS before the Self term and the stores.
template <int DP>
__global__ void __launch_bounds__(512) bwd_dq_kernel(const BwdParams p) {
  using E = Elem<bf16_t>;
  using Frag = E::Frag;
  constexpr int NW = 8;
  constexpr int DT = DP / 16, CPR = DP / 8, TILE = 64 * DP;
  constexpr int SLOT = TILE + 2 * 4096;   // bf16 per ring slot: the P2 tile, then each query block's 8 fragments
  constexpr int NS = 4;                   // ring slots: key blocks issued ahead + 1 (five measured slower)
  using Stager = TileStager<DP, NW, 1>;
  constexpr int PER = Stager::PER;        // P2 transfers per block of the busiest waves
  constexpr int RSF = DP + 4;             // fp32 row stride of the reduction buffer: an odd count of
                                          // 16-byte chunks, so a lane group's rows fall on distinct banks
  static_assert(128 * RSF * 4 <= NS * SLOT * 2, "the reduction buffer fits the ring");
  __shared__ __align__(16) bf16_t ring[NS * SLOT];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int li = lane & 15, lg = lane >> 4;
  const int kh = wave & 1, qq = wave >> 1;
  const int sub = qq >> 1, qh = qq & 1;
  const int BH = p.B * p.H;
  const int bh = blockIdx.x % BH;
  const int nqb = p.TQp / 64;
  const int qtop = nqb - 1 - 2 * (blockIdx.x / BH);  // the pair's later query block
  const bool wq = qtop - sub >= 0;                   // the wave has a query block (wave-uniform)
  const int qbw = wq ? qtop - sub : qtop;            // a wave without one mirrors the other's addresses
  const int b = bh / p.H, h = bh % p.H;
  const int ibase = (qtop - 1) * 64;                 // query of reduction row 0 (the earlier block)
  const bf16_t* kbase = reinterpret_cast<const bf16_t*>(p.p2) + b * p.k_sb + h * p.k_sh;
  const int nkb = PairTable::nkb(qtop, p.TQ, p.q_start);                   // the workgroup's key blocks
  const int nkb_w = PairTable::nkb(qbw, p.TQ, p.q_start);                  // the wave's (addresses)
  const int nkb_c = wq ? nkb_w : 0;                                        // the wave's (products)
  // the 2 KB of each pair that the key kernel's wave (kh, qh) stored
  const int fo = (kh * 4 + 2 * qh) * 512;
  const bf16_t* fr = reinterpret_cast<const bf16_t*>(p.dut) +
                     (int64_t(bh) * p.npairs + PairTable::offset(qbw, p.q_start)) * 4096 + fo + lane * 8;
  const int fslot = TILE + sub * 4096 + fo;  // the wave's fragments within a slot

  f32x4 dqacc[DT][2];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int s = 0; s < 2; ++s) dqacc[dt][s] = f32x4{0.f, 0.f, 0.f, 0.f};

  // The Self term's inputs, dU_ii and the P2 row of each of the thread's (query, 8-column chunk)
  // items, loaded before the key loop: their latency passes under it instead of after it. Rows
  // outside [0, TQ) load a row inside (not stored).
  constexpr int NIT = 128 * CPR / (64 * NW);
  static_assert(128 * CPR % (64 * NW) == 0, "whole (query, chunk) items per thread");
  float us_pre[NIT];
  Frag k8_pre[NIT];
#pragma unroll
  for (int it = 0; it < NIT; ++it) {
    const int item = tid + 64 * NW * it;
    const int i = min(max(ibase + item / CPR, 0), p.TQ - 1);
    us_pre[it] = p.duii[int64_t(bh) * p.TQp + i];
    k8_pre[it] = E::load8(kbase + int64_t(p.q_start + i) * p.k_sr + (item % CPR) * 8);
  }

  const bf16_t* srcs[1] = {kbase};
  const int64_t strides[1] = {p.k_sr};
  Stager st;
  st.init(wave, lane, strides);
  // Block kb: P2 rows (the staging instructions dealt over the waves) and the wave's fragments into
  // ring slot kb % NS, issued NS - 1 steps ahead; blocks past the end are not issued. A wave past its
  // own block's last key block reloads that block's last fragments (valid addresses, no products).
  // The wait before block kb's reads leaves in flight the later blocks already issued: NS - 2 of
  // them, fewer in the last steps; each wave counts its own transfers per block.
  auto issue = [&](int kb, auto u) {
    constexpr int U = decltype(u)::value;
    bf16_t* dst = ring + U * SLOT;
    st.issue(dst, srcs, strides, kb * 64, p.TK - 1, wave, lane);
    const int kc = min(kb, nkb_w - 1);
#pragma unroll
    for (int s = 0; s < 2; ++s) Stager::load(fr + int64_t(kc) * 4096 + s * 512, dst + fslot + s * 512);
  };
  const bool busy = wave + NW * (PER - 1) < Stager::NINS;  // this wave issues PER staging transfers, else PER - 1
  // wait until at most min(later, NS - 2) blocks of this wave's transfers are outstanding
  auto wait_blocks = [&](int later, auto vms) {
    constexpr int V = decltype(vms)::value;
    static_assert(NS >= 3 && NS <= 6, "ring depth");
    if (later >= NS - 2) __builtin_amdgcn_s_waitcnt(kVmWaitStage<(NS - 2) * V>());
    else if (NS > 5 && later == 3) __builtin_amdgcn_s_waitcnt(kVmWaitStage<(NS > 5 ? 3 : 0) * V>());
    else if (NS > 4 && later == 2) __builtin_amdgcn_s_waitcnt(kVmWaitStage<(NS > 4 ? 2 : 0) * V>());
    else if (NS > 3 && later == 1) __builtin_amdgcn_s_waitcnt(kVmWaitStage<(NS > 3 ? 1 : 0) * V>());
    else __builtin_amdgcn_s_waitcnt(kVmWaitStage<0>());
  };
  auto wait_for = [&](int later) {
    if (busy) wait_blocks(later, std::integral_constant<int, PER + 2>{});
    else wait_blocks(later, std::integral_constant<int, PER + 1>{});
  };
  auto step = [&](int kb, auto u) {
    constexpr int U = decltype(u)::value;
    if (kb >= nkb) return;  // uniform over the workgroup: every wave skips the same steps
    wait_for(nkb - 1 - kb);  // this wave's part of block kb is in
    lds_barrier();  // every wave's part of block kb is in; every wave is done with block kb - 1's slot
    if (kb + NS - 1 < nkb) issue(kb + NS - 1, std::integral_constant<int, (U + NS - 1) % NS>{});
    if (kb >= nkb_c) return;  // wave-uniform: the earlier block has no pair with this key block
    const bf16_t* Ks = ring + U * SLOT;
    Frag bf[2];
#pragma unroll
    for (int s = 0; s < 2; ++s) bf[s] = dut_frag(Ks + fslot, s, li, lg);
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      const Frag ak = tile_tr_frag<DP>(Ks, 32 * kh, dt, li, lg);
#pragma unroll
      for (int s = 0; s < 2; ++s) dqacc[dt][s] = E::mma(ak, bf[s], dqacc[dt][s]);
    }
  };
  if (nkb > 0) {
    static_for<NS - 1>([&](auto u) {
      if (decltype(u)::value < nkb) issue(decltype(u)::value, u);
    });
    for (int kb0 = 0; kb0 < nkb; kb0 += NS) static_for<NS>([&](auto u) { step(kb0 + decltype(u)::value, u); });
  }

  // add the two key halves through LDS: [128 queries][RSF] fp32 over the ring, rows 0..63 the
  // earlier block, 64..127 the later one
  float* R = reinterpret_cast<float*>(ring);
  const int rbase = (1 - sub) * 64 + 32 * qh;
  __syncthreads();  // every wave is done reading the ring (the last step waited for every transfer)
  if (kh == 1) {
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int s = 0; s < 2; ++s)
        *reinterpret_cast<f32x4*>(R + (rbase + 16 * s + li) * RSF + 16 * dt + 4 * lg) = dqacc[dt][s];
  }
  __syncthreads();
  if (kh == 0) {
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        f32x4* q = reinterpret_cast<f32x4*>(R + (rbase + 16 * s + li) * RSF + 16 * dt + 4 * lg);
        *q = *q + dqacc[dt][s];
      }
  }
  __syncthreads();
  // Self part dU_ii P2_i, scale, 16-byte stores
  bf16_t* dqout = reinterpret_cast<bf16_t*>(p.dp1) + b * p.dq_sb + h * p.dq_sh;
#pragma unroll
  for (int it = 0; it < NIT; ++it) {
    const int item = tid + 64 * NW * it;
    const int row = item / CPR, d0 = (item % CPR) * 8;
    const int i = ibase + row;
    if (i < 0 || i >= p.TQ) continue;
    const float us = us_pre[it];
    const Frag k8 = k8_pre[it];
    float o[8];
#pragma unroll
    for (int e = 0; e < 8; e += 4) {
      const float4 a = *reinterpret_cast<const float4*>(R + row * RSF + d0 + e);
      o[e] = a.x; o[e + 1] = a.y; o[e + 2] = a.z; o[e + 3] = a.w;
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = fmaf(us, (float)k8.v[e], o[e]) * p.scale;
    const Frag ov = E::from_f32(o);
    *reinterpret_cast<bf16x8*>(dqout + int64_t(i) * p.dq_sr + d0) = ov.v;
  }
  // the last workgroup (the lowest pair, the shortest) also sums dlam: the rows stage has written
  // every partial before this launch
  if (blockIdx.x == gridDim.x - 1) {
    __syncthreads();  // the Self-term reads of R are done before dlam_sum reuses the memory
    dlam_sum<64 * NW>(p.dlam_part, BH * nqb, p.dlam, R);
  }
}

// ------------------------------------------------------------------------------------------------
// host side
// ------------------------------------------------------------------------------------------------
template <int DP>
static void launch_tiles_dp(const BwdParams& p, int stages, hipStream_t stream) {
  const int BH = p.B * p.H;
  if (stages & MOTE_BWD_KEYS) {
    const int nkb = (p.TK + 63) / 64;
    hipLaunchKernelGGL((bwd_kv_kernel<DP>), dim3(nkb * BH), dim3(256), 0, stream, p);
  }
  if (stages & MOTE_BWD_QUERIES) {
    const int npq = (p.TQp / 64 + 1) / 2;  // query-block pairs
    hipLaunchKernelGGL((bwd_dq_kernel<DP>), dim3(npq * BH), dim3(512), 0, stream, p);
  }
}

void launch_bwd_tiles(const BwdParams& p, int stages, hipStream_t stream) {
  switch (p.D) {
    case 32: launch_tiles_dp<32>(p, stages, stream); break;
    case 64: launch_tiles_dp<64>(p, stages, stream); break;
    case 96: launch_tiles_dp<96>(p, stages, stream); break;
    default: launch_tiles_dp<128>(p, stages, stream); break;
  }
}

}  // namespace mote
