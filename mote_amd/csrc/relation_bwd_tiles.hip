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
#include <atomic>
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

// The fused launch (bwd_kvq_kernel) stores dU write-through: buffer stores with the SC1 cache-policy
// bit (agent scope), so once the storing wave's s_waitcnt has seen them complete they are at the
// device-coherent level, where the query work of any XCD reads them with SC1 loads (no stale line of
// its own L2). Byte offsets past the buffer's range are dropped by the hardware.
typedef __attribute__((ext_vector_type(4))) unsigned int u32x4;
constexpr int kCpolSc1 = 16;          // cache-policy operand of the buffer builtins: SC1
constexpr int kBufWord3 = 0x00020000; // buffer resource word 3 of the gfx9 family: 32-bit data format

__device__ __forceinline__ void store16_wt(__amdgpu_buffer_rsrc_t rs, uint32_t off, const bf16x8& v) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), rs, off, 0, kCpolSc1);
}

// store_dut / store_dut_zero through the write-through stores; `off` = byte offset of the wave's 2 KB
__device__ __forceinline__ void store_dut_wt(const Elem<bf16_t>::Frag (&au)[2], __amdgpu_buffer_rsrc_t rs, uint32_t off,
                                             int lane) {
  const uint32_t o = off + uint32_t(dut_pos(lane)) * 16u;
  store16_wt(rs, o, au[0].v);
  store16_wt(rs, o + 1024u, au[1].v);
}

__device__ __forceinline__ void store_dut_zero_wt(__amdgpu_buffer_rsrc_t rs, uint32_t off, int lane) {
  store16_wt(rs, off + uint32_t(lane) * 16u, bf16x8{});
  store16_wt(rs, off + 1024u + uint32_t(lane) * 16u, bf16x8{});
}

// ------------------------------------------------------------------------------------------------
// key-stationary kernel: dP2 and dI~
// ------------------------------------------------------------------------------------------------
template <int DP, bool MASKED, bool WT>
__device__ __forceinline__ void kv_block(const bf16_t* Qs, const bf16_t* Ds, const float* Ss, const bf16_t* Ks,
                                         const bf16_t* Vs, f32x4 (&dvacc)[2][DP / 16], f32x4 (&dkacc)[2][DP / 16],
                                         bf16_t* dut_w, __amdgpu_buffer_rsrc_t rs, uint32_t dut_b, int qh, int kh,
                                         int li, int lg, int key0, int qa0, float nc2) {
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
  if (dut_w) {
    if constexpr (WT)
      store_dut_wt(au, rs, dut_b, lane_of(li, lg));
    else
      store_dut(au, dut_w, lane_of(li, lg));
  }
}

template <int DP>
struct KvShape {
  static constexpr int TILE = 64 * DP;
  static constexpr int STAGE = 2 * TILE + 256;     // bf16 slots per stage: Q tile, dI-bar tile, 128 fp32 stats
  static constexpr int LDS = 2 * STAGE + 2 * TILE;  // two stages, then the job's 64 P2 rows and 64 I~ rows
};

// The key work of one (batch x head) bh and key block kb: 64 keys, 4 waves. FUSED (the fused launch):
// the query blocks are walked from the last down, so the pairs of the longest query blocks are stored
// first, and the dU quadrants of each query block are counted in the kvq counts once stored.
template <int DP, bool FUSED>
__device__ __forceinline__ void kv_job(const BwdParams& p, const int bh, const int kb, bf16_t* smem) {
  using E = Elem<bf16_t>;
  using Frag = E::Frag;
  using S = KvShape<DP>;
  constexpr int DT = DP / 16, CPR = DP / 8, TILE = S::TILE, STAGE = S::STAGE;
  bf16_t* kvs = smem + 2 * STAGE;  // the job's 64 P2 rows, then its 64 I~ rows

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: staging in scalar registers
  const int li = lane & 15, lg = lane >> 4;
  const int kh = wave & 1, qh = wave >> 1;
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
  const int qb_lo = max(0, k0 + 1 - p.q_start) / 64;  // the first query block that sees a key of the block
  const int qb_first = FUSED ? nqb - 1 : qb_lo;        // the walk's first block
  // PairTable::offset(qb) for the block in hand, moved by qb + A per block (offset(qb + 1) - offset(qb))
  const int pair_a = (p.q_start + 126) / 64;
  int64_t pair_off = PairTable::offset(qb_first, p.q_start);
  // dU of this key block: pair (qb, kb) at PairTable::offset(qb) + kb, 8 KB per pair; wave (kh, qh)
  // writes its 2 KB at (kh * 4 + 2 qh) * 512 elements (store_dut)
  const int wq_off = (kh * 4 + 2 * qh) * 512;
  bf16_t* dut_bh = reinterpret_cast<bf16_t*>(p.dut) + int64_t(bh) * p.npairs * 4096 + wq_off;
  // FUSED: the (batch x head)'s pairs as one buffer (the host keeps it below 2^31 bytes)
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
      reinterpret_cast<bf16_t*>(p.dut) + int64_t(bh) * p.npairs * 4096, 0, int(p.npairs * 8192), kBufWord3);
  int* const cnt = FUSED ? p.kvq + kKvqCounts + bh * nqb : nullptr;
  {
    // the key rows once (rows past the keys: finite copies whose results are never stored)
    const bf16_t* ksrc[2] = {kbase, vbase};
    const int64_t kstr[2] = {p.k_sr, p.v_sr};
    TileStager<DP, 4, 2> kst;
    kst.init(wave, lane, kstr);
    kst.issue(kvs, ksrc, kstr, k0, p.TK - 1, wave, lane);
  }
  if (qb_lo < nqb) issue(qb_first, 0);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  // FUSED: the count of a block's four dU quadrants is one atomic add by wave 0, issued right after
  // the transfers two blocks later: the waits of the next two blocks leave it in flight, so it costs
  // no wait of its own (an add waited for at the end of the next block, against the transfers, ran
  // the key work 20 % slower). `prev`: the block of the previous step (its stores in flight);
  // `ready`: the block before (every wave's stores seen complete before the previous barrier).
  int prev = -1, ready = -1;
  // Diagonal query blocks (some key not before some query) with the masked block math, the rest
  // with the unmasked math: two loops instead of a branch keeps one register assignment of the
  // accumulators per loop.
  auto step = [&](int qb, auto masked) {
    const int n = FUSED ? nqb - 1 - qb : qb - qb_lo;  // position in the walk
    MOTE_STAMP(0, n);
    const int stage = n & 1;
    const int qn = FUSED ? qb - 1 : qb + 1;  // the walk's next block
    if (FUSED ? qn >= qb_lo : qn < nqb) issue(qn, stage ^ 1);
    bool sig = false;  // wave 0 added a count after the transfers (one more operation in flight)
    if constexpr (FUSED) {
      sig = wave == 0 && ready >= 0;
      asm volatile("" ::: "memory");  // the add after the transfers, in issue order
      if (sig && lane == 0) __hip_atomic_fetch_add(cnt + ready, 4, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    MOTE_STAMP(1, n);
    const bf16_t* Qs = smem + stage * STAGE;
    const bf16_t* Ds = Qs + TILE;
    const float* Ss = reinterpret_cast<const float*>(Qs + 2 * TILE);
    const int i0 = qb * 64 + 32 * qh;   // the wave's first query row
    const int qa0 = p.q_start + i0;     // its position
    const bool pair = kb < PairTable::nkb(qb, p.TQ, p.q_start);
    bf16_t* dut_w = pair ? dut_bh + (pair_off + kb) * 4096 : nullptr;
    const uint32_t dut_b = uint32_t(pair_off + kb) * 8192u + uint32_t(wq_off) * 2u;
    pair_off += FUSED ? -int64_t(qb - 1 + pair_a) : int64_t(qb + pair_a);  // PairTable::offset(qn)
    // quadrant visible at all (some key < some query position), and not wholly padding rows
    if (i0 < p.TQ && key0 < qa0 + 31)
      kv_block<DP, decltype(masked)::value, FUSED>(Qs, Ds, Ss, kvs, kvs + TILE, dvacc, dkacc, dut_w, rs, dut_b, qh,
                                                   kh, li, lg, key0, qa0, nc2);
    else if (dut_w) {
      if constexpr (FUSED)
        store_dut_zero_wt(rs, dut_b, lane);
      else
        store_dut_zero(dut_w, lane);
    }
    MOTE_STAMP(2, n);
    // The next block's transfers were issued before this block's two dU^T stores (and the count's
    // add), and vector-memory operations retire in issue order: waiting until at most those are
    // outstanding means the transfers have landed, while the stores stay in flight across the
    // barrier. Everything issued before the transfers has completed too: the previous block's stores.
    if (dut_w) {
      if (sig)
        __builtin_amdgcn_s_waitcnt(kVmWaitStage<3>());
      else
        __builtin_amdgcn_s_waitcnt(kVmWaitStage<2>());
    } else {
      if (sig)
        __builtin_amdgcn_s_waitcnt(kVmWaitStage<1>());
      else
        __builtin_amdgcn_s_waitcnt(kVmWaitStage<0>());
    }
    MOTE_STAMP(3, n);
    lds_barrier();
    MOTE_STAMP(4, n);
    if constexpr (FUSED) {
      ready = prev;
      prev = pair ? qb : -1;
    }
  };
  // unmasked for every wave once the block's first query position exceeds the last key
  const int qb_m = min(nqb, max(qb_lo, k0 + 63 - p.q_start >= 0 ? (k0 + 63 - p.q_start) / 64 + 1 : 0));
  if constexpr (FUSED) {
    for (int qb = nqb - 1; qb >= qb_m; --qb) step(qb, std::false_type{});
    for (int qb = qb_m - 1; qb >= qb_lo; --qb) step(qb, std::true_type{});
    // the last two blocks: every wave's stores complete, then their counts
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (wave == 0 && lane == 0) {
      if (ready >= 0) __hip_atomic_fetch_add(cnt + ready, 4, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (prev >= 0) __hip_atomic_fetch_add(cnt + prev, 4, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  } else {
    int qb = qb_lo;
    for (; qb < qb_m; ++qb) step(qb, std::true_type{});
    for (; qb < nqb; ++qb) step(qb, std::false_type{});
  }

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

template <int DP>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(DP <= 96 ? 2 : 1)))
bwd_kv_kernel(const BwdParams p) {
  __shared__ __align__(16) bf16_t smem[KvShape<DP>::LDS];
  const int BH = p.B * p.H;
  kv_job<DP, false>(p, blockIdx.x % BH, blockIdx.x / BH, smem);  // key block 0 sees the most queries: longest first
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
// The fused launch runs the same work as a four-wave job of one query block (NW = 4), after a wait
// for the counts of its pairs' dU quadrants, reading the quadrants with SC1 loads.
template <int DP, int NW>
struct DqShape {
  static constexpr int NQB = NW / 4;                // query blocks per job
  static constexpr int TILE = 64 * DP;
  static constexpr int SLOT = TILE + NQB * 4096;    // bf16 per ring slot: the P2 tile, then each query block's 8 fragments
  static constexpr int NS = NW == 8 ? 4 : 3;        // ring slots: key blocks issued ahead + 1 (five measured slower)
  static constexpr int LDS = NS * SLOT;
};

template <int DP, int NW, bool FUSED>
__device__ __forceinline__ void dq_job(const BwdParams& p, const int bh, const int qtop, bf16_t* ring) {
  using E = Elem<bf16_t>;
  using Frag = E::Frag;
  using Q = DqShape<DP, NW>;
  static_assert(!FUSED || NW == 4, "the fused launch runs four-wave jobs");
  constexpr int NQB = Q::NQB, SLOT = Q::SLOT, NS = Q::NS;
  constexpr int DT = DP / 16, CPR = DP / 8, TILE = Q::TILE;
  using Stager = TileStager<DP, NW, 1>;
  constexpr int PER = Stager::PER;        // P2 transfers per block of the busiest waves
  constexpr int RSF = DP + 4;             // fp32 row stride of the reduction buffer: an odd count of
                                          // 16-byte chunks, so a lane group's rows fall on distinct banks
  static_assert(64 * NQB * RSF * 4 <= NS * SLOT * 2, "the reduction buffer fits the ring");

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int li = lane & 15, lg = lane >> 4;
  const int kh = wave & 1, qq = wave >> 1;
  const int sub = qq >> 1, qh = qq & 1;
  const int nqb = p.TQp / 64;
  const bool wq = qtop - sub >= 0;                   // the wave has a query block (wave-uniform)
  const int qbw = wq ? qtop - sub : qtop;            // a wave without one mirrors the other's addresses
  const int b = bh / p.H, h = bh % p.H;
  const int ibase = (qtop - (NQB - 1)) * 64;         // query of reduction row 0 (the earlier block)
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
  constexpr int NIT = 64 * NQB * CPR / (64 * NW);
  static_assert(64 * NQB * CPR % (64 * NW) == 0, "whole (query, chunk) items per thread");
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
    for (int s = 0; s < 2; ++s) {
      if constexpr (FUSED)
        lds_dma16_sc1(fr + int64_t(kc) * 4096 + s * 512, dst + fslot + s * 512);
      else
        Stager::load(fr + int64_t(kc) * 4096 + s * 512, dst + fslot + s * 512);
    }
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
  bool overrun = false;  // FUSED: the wait gave up; the job then writes its dP1 rows as NaN
  if constexpr (FUSED) {
    // every pair of the query block counted (four quadrants each) before any of its dU is read; the
    // key work of every pair was taken from the job counter before this job, so each count completes
    __shared__ int s_over;
    if (tid == 0) {
      int* c = p.kvq + kKvqCounts + bh * nqb + qtop;
      int over = 0;
      const int target = 4 * nkb + p.kvq_extra;
      for (int spin = 0;; ++spin) {
        const int have = __hip_atomic_load(c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (have >= target) break;
        if (spin >= p.kvq_spin) {
          over = 1;
          break;
        }
        // about 3.5 us between polls while more than two pairs are missing (polls every ~1 us by all
        // the waiting jobs held up the key work's count adds: 30-60 % slower at 2-3 K rows), a few
        // hundred ns once the block is nearly complete (the launch's last jobs: 1.5 % shorter at C3)
        if (target - have <= 8)
          __builtin_amdgcn_s_sleep(8);
        else
          __builtin_amdgcn_s_sleep(127);
      }
      s_over = over;
    }
    __syncthreads();
    overrun = s_over != 0;
  }
  if (nkb > 0 && !overrun) {
    static_for<NS - 1>([&](auto u) {
      if (decltype(u)::value < nkb) issue(decltype(u)::value, u);
    });
    for (int kb0 = 0; kb0 < nkb; kb0 += NS) static_for<NS>([&](auto u) { step(kb0 + decltype(u)::value, u); });
  }

  // add the two key halves through LDS: [64 NQB queries][RSF] fp32 over the ring, rows 0..63 the
  // earlier block, 64..127 the later one
  float* R = reinterpret_cast<float*>(ring);
  const int rbase = (NQB - 1 - sub) * 64 + 32 * qh;
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
    for (int e = 0; e < 8; ++e) o[e] = overrun ? __builtin_nanf("") : fmaf(us, (float)k8.v[e], o[e]) * p.scale;
    const Frag ov = E::from_f32(o);
    *reinterpret_cast<bf16x8*>(dqout + int64_t(i) * p.dq_sr + d0) = ov.v;
  }
}

template <int DP>
__global__ void __launch_bounds__(512) bwd_dq_kernel(const BwdParams p) {
  __shared__ __align__(16) bf16_t ring[DqShape<DP, 8>::LDS];
  const int BH = p.B * p.H, nqb = p.TQp / 64;
  dq_job<DP, 8, false>(p, blockIdx.x % BH, nqb - 1 - 2 * (blockIdx.x / BH), ring);  // the pair's later query block
  // the last workgroup (the lowest pair, the shortest) also sums dlam: the rows stage has written
  // every partial before this launch
  if (blockIdx.x == gridDim.x - 1) {
    __syncthreads();  // the Self-term reads of the ring are done before dlam_sum reuses the memory
    dlam_sum<512>(p.dlam_part, BH * nqb, p.dlam, reinterpret_cast<float*>(ring));
  }
}

// ------------------------------------------------------------------------------------------------
// fused key + query launch
// ------------------------------------------------------------------------------------------------
// One launch of four-wave workgroups for both kinds of work: as many workgroups as fit the GPU at
// once (two per CU), each taking jobs until its queue is empty. The (batch x head)s are dealt over
// kvq_nq queues (head bh to queue bh % kvq_nq), each with its own job counter, and workgroup i takes
// its jobs from queue i % kvq_nq: first the queue's key jobs (key blocks, longest first), then its
// query jobs (query blocks, longest first). Workgroups are dealt round-robin over the 8 XCDs, so a
// queue's jobs run on the XCDs i % 8 = queue (mod kvq_nq), whose L2s then hold their heads' query
// tiles, as in the two-launch form. A query job waits until the dU quadrants of all its pairs are
// counted; the key jobs it waits on are in its own queue and were taken before it by running
// workgroups, which never wait, so every wait ends. The query work of the long query blocks runs
// beside the key work's tail (key block 0's walk, the launch's longest chain), in the slots the key
// work no longer fills. (With one job per workgroup instead, the dispatcher places workgroups in
// order, round-robin over the XCDs, and one XCD without a free slot holds back every later
// workgroup: a third of the slots stood empty through the second half of the launch.)
template <int DP>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) bwd_kvq_kernel(const BwdParams p) {
  constexpr int LDS = KvShape<DP>::LDS > DqShape<DP, 4>::LDS ? KvShape<DP>::LDS : DqShape<DP, 4>::LDS;
  static_assert(LDS * 2 <= 80 * 1024, "two workgroups per CU");
  __shared__ __align__(16) bf16_t lds[LDS];
  __shared__ int s_job;
  const int nq = p.kvq_nq, queue = blockIdx.x % nq;
  const int BH = p.B * p.H, hq = BH / nq, nqb = p.TQp / 64;  // hq heads per queue
  const int nkey = (p.TK + 63) / 64 * hq, nqj = nqb * hq;
  for (;;) {
    if (threadIdx.x == 0)
      s_job = __hip_atomic_fetch_add(p.kvq + kKvqJob + queue * kKvqJobStride, 1, __ATOMIC_RELAXED,
                                     __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    const int job = __builtin_amdgcn_readfirstlane(s_job);
    if (job >= nkey + nqj) break;
    if (job < nkey) {
      kv_job<DP, true>(p, queue + nq * (job % hq), job / hq, lds);
    } else {
      const int j = job - nkey;
      dq_job<DP, 4, true>(p, queue + nq * (j % hq), nqb - 1 - j / hq, lds);
      if (queue == 0 && j == nqj - 1) {
        // queue 0's last job (its shortest) also sums dlam: the rows stage has written every partial
        __syncthreads();
        dlam_sum<256>(p.dlam_part, BH * nqb, p.dlam, reinterpret_cast<float*>(lds));
      }
    }
    __syncthreads();  // the next job reuses the LDS and s_job
  }
}

// ------------------------------------------------------------------------------------------------
// host side
// ------------------------------------------------------------------------------------------------
// compute units of the current device (read once per device)
int device_cu_count() {
  static std::atomic<int> cus[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  int n = cus[dev].load(std::memory_order_relaxed);
  if (n <= 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cus[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

// the fused launch's control words when no rows stage in the same call has cleared them
__global__ void __launch_bounds__(256) kvq_clear_kernel(int* kvq, int n) {
  for (int i = blockIdx.x * 256 + threadIdx.x; i < n; i += gridDim.x * 256)
    __hip_atomic_store(kvq + i, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int DP>
static void launch_tiles_dp(const BwdParams& p, int stages, hipStream_t stream) {
  const int BH = p.B * p.H;
  if constexpr (DP <= 96) {
    if (p.kvq && (stages & MOTE_BWD_KEYS) && (stages & MOTE_BWD_QUERIES)) {
      const int nqb = p.TQp / 64, nkb = (p.TK + 63) / 64;
      if (!(stages & MOTE_BWD_ROWS)) {
        const int n = kKvqCounts + BH * nqb;
        hipLaunchKernelGGL(kvq_clear_kernel, dim3((n + 255) / 256 < 64 ? (n + 255) / 256 : 64), dim3(256), 0, stream,
                           p.kvq, n);
      }
      // at most as many workgroups as are resident at once (two per CU), a multiple of the queue
      // count. Workgroups beyond the key jobs take query jobs at once and wait in their slots for the
      // key work; that pays only while the key walks are short: with 12 or more query blocks the grid
      // is the key jobs alone (H 8 at 2048 rows: 68 against 81-91 us with one workgroup per job; at
      // 300-700 rows one per job measured 0.5-1.2 us faster)
      const int resident = 2 * device_cu_count();
      const int jobs = nqb >= 12 ? nkb * BH : (nkb + nqb) * BH;
      const int grid = (jobs < resident ? jobs : resident) / p.kvq_nq * p.kvq_nq;
      hipLaunchKernelGGL((bwd_kvq_kernel<DP>), dim3(grid > 0 ? grid : p.kvq_nq), dim3(256), 0, stream, p);
      return;
    }
  }
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
