// Fused projection prologue of FullRelation (mote/model/relation.py:199-215): the QKV product
// x [w1; w2; wi]^T with RoPE on p1 / p2 and the Givens head-pair rotation on I~ in its epilogue,
// written straight into the [B, T, H, dh] layout the Relation kernels and the arena read.
//
// Product. C^T = W X^T on v_mfma_f32_16x16x32_bf16: a workgroup (4 waves at dh 64 / 96, 8 at dh 128)
// owns 32 tokens per wave and the 2 dh output features of one head pair of one projection (p1, p2:
// heads 2k, 2k+1; I~: the Givens pair of the layer's parity, (2k, 2k+1) or (2k+1, 2k+2 mod H)). Wave
// w holds head (w & 1) for tokens 64 (w >> 1) .. +63: dh/16 x 4 accumulator tiles, features in the
// rows, tokens in the columns, so a lane ends with 4 consecutive features of one token. At dh 64 / 96
// a workgroup needs 64 / 80 KB of LDS and at most 256 registers a lane, so two share a CU and one's
// epilogue (rounding, rotations, stores: about 40 % of a workgroup's time) overlaps the other's
// products; 256 tokens per workgroup (8 waves) left one workgroup per CU and the CU's matrix cores
// idle through every epilogue (417 against 374 us at 79,424 rows, dh 96). At dh 128 four waves would
// still leave one workgroup per CU (98 KB of LDS, 272 registers), so it keeps eight.
// k advances 64 at a time through two LDS slots filled by direct global -> LDS transfers (8 token or
// weight rows x 128 bytes per wave instruction, chunks XOR-swizzled within a row): after the stage's
// barrier a wave reads all of its fragments of the stage at once (one LDS latency per stage), issues
// the next stage's transfers into the other slot, then runs the products. 128 x 2 dh outputs per
// stage keep the L2 -> LDS traffic at about 77 flop per byte (dh 96).
//
// Epilogue. The product, rounded to bf16 (the projection output the reference rotates), goes to a
// padded LDS tile [tokens][2 dh]; then every thread takes pairs of 16-byte chunks of it (RoPE:
// chunk c and c + dh/16 of one head, the two halves that rotate together, relation.py:53-58; Givens:
// the same chunk of the pair's two heads, :160-174) and stores both rotated chunks,
// out_a = a C - b S, out_b = b C + a S, with C, S the bf16-rounded factors (cos / sin of
// float(pos) * inv_freq[k] from a table kernel: one table entry serves both chunks of a RoPE pair;
// cos / sin of theta), exactly as the unfused rope_givens kernels compute them. Optionally the
// pre-rotation I~ is kept for the backward (d theta).
#include "common.hpp"
#include "params.hpp"
#include "tiles.hpp"

namespace mote {

// waves per workgroup: a wave pair covers 64 tokens of both heads (64 tokens x dh per wave; 4 waves
// with 128 x dh per wave hold their accumulators in AGPRs at one wave per SIMD: slower)
template <int DH>
constexpr int qkv_waves() { return DH == 128 ? 8 : 4; }
constexpr int kQkvK = 64;        // k per stage (a 128-byte line of every staged row)
constexpr int kQkvStg = 2;       // ring depth
constexpr int kQkvPad = 8;       // bf16 elements of padding per output-tile row

struct QkvParams {
  const bf16_t* x; int64_t x_sr;           // [M, K] token rows (M = B * T)
  const bf16_t* w; int64_t w_sr;           // [3 H dh, K]
  const uint32_t* tab;                     // [T][dh / 2] bf16 cos | bf16 sin << 16, or null (no RoPE)
  const float* theta;                      // [H / 2] or null (no Givens)
  bf16_t* o1; int64_t o1_sb, o1_sh, o1_sr;
  bf16_t* o2; int64_t o2_sb, o2_sh, o2_sr;
  bf16_t* o3; int64_t o3_sb, o3_sh, o3_sr;
  bf16_t* iraw; int64_t ir_sb, ir_sr;      // [B, T, H dh] pre-rotation I~, or null
  const float* nw1;                        // QK-Norm gains [dh] of p1 / p2 (fp32), or null: no QK-Norm
  const float* nw2;
  float eps;
  bf16_t* qkraw; int64_t qr_sb, qr_sr;     // [B, T, 2 H dh] p1 | p2 projections before QK-Norm, or null
  const bf16_t* gy; int64_t gy_sr;         // gate mode: y [M, H dh] (the Relation output, token-major)
  bf16_t* gz; bf16_t* gs; int64_t gz_sr;   // gate mode: z = y sigmoid(x wg^T) and the sigmoid, [M, H dh]
  int B, T, H, K, M, parity, nk;
  int ntok, ncol;                          // token tiles, column tiles (3 H / 2)
};

template <int DH, int NW>
struct QkvShape {
  static constexpr int TOK = 32 * NW;                 // tokens per workgroup
  static constexpr int NF = DH / 16;                  // feature tiles per head
  static constexpr int TPW = TOK / (NW / 2);          // tokens per wave (waves pair up over the two heads)
  static constexpr int NT = TPW / 16;                 // token tiles per wave
  static constexpr int ROWS = 2 * DH + TOK;           // staged rows per stage: W head 0 | W head 1 | X
  static constexpr int CPR = kQkvK / 8;              // 16-byte chunks per staged row
  static constexpr int RPI = 64 / CPR;                // rows per wave instruction
  static constexpr int NINS = ROWS / RPI;             // wave instructions per stage
  static constexpr int PER = (NINS + NW - 1) / NW;   // per wave (waves >= NINS % NW issue one
  static constexpr int FULL = NINS % NW == 0 ? NW : NINS % NW;  // fewer when NINS % NW != 0)
  static constexpr int STAGE = ROWS * kQkvK;          // bf16 elements
  static constexpr int OUTW = 2 * DH + kQkvPad;
  static constexpr int NCH = 2 * DH / 8;              // 16-byte chunks per output-tile row
  static constexpr int LDS = kQkvStg * STAGE > TOK * OUTW ? kQkvStg * STAGE : TOK * OUTW;
};

// rope table: tab[t][k] = bf16(cos a) | bf16(sin a) << 16, a = float(pos0 + t) * inv_freq[k]
__global__ void __launch_bounds__(256) rope_table_kernel(const float* inv_freq, int pos0, int T, int half,
                                                         uint32_t* tab) {
  const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (i >= int64_t(T) * half) return;
  const int t = int(i / half), k = int(i % half);
  float sn, cs;
  sincosf((float)(pos0 + t) * inv_freq[k], &sn, &cs);
  tab[i] = uint32_t(f2bf(cs)) | (uint32_t(f2bf(sn)) << 16);
}

template <int DH, int NW, bool GATE>
__global__ void __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(2)))
qkv_rope_kernel(const QkvParams p) {
  using S = QkvShape<DH, NW>;
  using E = Elem<bf16_t>;
  __shared__ __align__(16) bf16_t smem[S::LDS];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // workgroup id -> (token tile, column tile): workgroups go round-robin over the 8 XCDs, so XCD j
  // takes the j-th contiguous run of the (token tile, column) order: a few token tiles with all their
  // column tiles, which its L2 holds while they are in use
  const int nwg = p.ntok * p.ncol, per = (nwg + 7) / 8;
  const int seq = (blockIdx.x % 8) * per + blockIdx.x / 8;
  if (seq >= nwg) return;
  const int r0 = (seq / p.ncol) * S::TOK;
  const int colt = seq % p.ncol;
  const int npair = p.H / 2;
  const int part = GATE ? 0 : colt / npair, hp = GATE ? colt : colt % npair;
  int h0 = 2 * hp, h1 = 2 * hp + 1;
  if (part == 2 && p.parity) {
    h0 = 2 * hp + 1;
    h1 = (2 * hp + 2) % p.H;
  }
  const int HD = p.H * DH;
  const bf16_t* wb0 = p.w + int64_t(part * HD + h0 * DH) * p.w_sr;
  const bf16_t* wb1 = p.w + int64_t(part * HD + h1 * DH) * p.w_sr;
  const bf16_t* xb = p.x + int64_t(r0) * p.x_sr;
  const bool full = r0 + S::TOK <= p.M;

  // staging: instruction g covers stage rows RPI g .. RPI g + RPI - 1; lane l takes row RPI g + l / CPR
  // and physical chunk l % CPR, i.e. logical chunk (l % CPR) ^ tile_swz(row). The lane offsets hold the
  // row within the source tile too (strides below 2^23 elements keep them in 32 bits), so a stage
  // issues from three scalar bases: the two weight heads and the token rows.
  constexpr int GW = DH / S::RPI;  // instructions per weight head
  const int lrow = lane / S::CPR;
  uint32_t voff[S::PER];
  int lchs[S::PER];
#pragma unroll
  for (int i = 0; i < S::PER; ++i) {
    const int g = wave + NW * i;
    const int64_t sr = g < 2 * GW ? p.w_sr : p.x_sr;
    const int lch = (lane % S::CPR) ^ tile_swz<kQkvK>(S::RPI * g + lrow);
    lchs[i] = lch;
    const int trow = g < GW ? S::RPI * g : (g < 2 * GW ? S::RPI * (g - GW) : S::RPI * (g - 2 * GW));
    voff[i] = uint32_t((trow + lrow) * int(sr) + lch * 8) * 2u;
  }
  const bool more = wave < S::FULL;  // this wave issues PER transfers per stage (else PER - 1)
  // transfer i of the wave's share of stage kb into ring slot `slot` (forced inline: at PER 10 the
  // compiler otherwise makes the lambdas calls and their scalar operands VGPR arguments)
  auto issue_i = [&](int i, int kb, int slot) __attribute__((always_inline)) {
    const int g = wave + NW * i;
    if (i == S::PER - 1 && !more) return;
    kb = min(kb, p.nk - 1);  // past the end: the last stage again (keeps every wave's count equal)
    const int k0 = kb * kQkvK;
    bf16_t* d = smem + slot * S::STAGE + g * 512;
    if (g < GW) {
      lds_dma16_s(wb0 + k0, voff[i], d);
    } else if (g < 2 * GW) {
      lds_dma16_s(wb1 + k0, voff[i], d);
    } else if (full) {
      lds_dma16_s(xb + k0, voff[i], d);
    } else {
      const int r = min(r0 + S::RPI * (g - 2 * GW) + lrow, p.M - 1);
      lds_dma16(p.x + int64_t(r) * p.x_sr + k0 + lchs[i] * 8, d);
    }
  };
  auto issue = [&](int kb, int slot) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < S::PER; ++i) issue_i(i, kb, slot);
  };

  const int hw = wave & 1, tw = wave >> 1;
  f32x4 acc[S::NF][S::NT];
#pragma unroll
  for (int f = 0; f < S::NF; ++f)
#pragma unroll
    for (int t = 0; t < S::NT; ++t) acc[f][t] = f32x4{0.f, 0.f, 0.f, 0.f};

#pragma unroll
  for (int i = 0; i < kQkvStg - 1; ++i) issue(i, i);
  int slot = 0;
  for (int kb = 0; kb < p.nk; ++kb) {
    // stage kb is complete once at most kQkvStg - 2 younger stages of this wave are outstanding
    if (kQkvStg == 2) __builtin_amdgcn_s_waitcnt(0);
    else if (more) __builtin_amdgcn_s_waitcnt(kVmWaitStage<(kQkvStg - 2) * S::PER>());
    else __builtin_amdgcn_s_waitcnt(kVmWaitStage<(kQkvStg - 2) * (S::PER - 1)>());
    lds_barrier();
    const int nslot = slot == 0 ? kQkvStg - 1 : slot - 1;
    const bf16_t* st = smem + slot * S::STAGE;
    // every fragment of the stage first (one LDS latency per stage), the next stage's transfers,
    // then the products
    constexpr int KK = kQkvK / 32;
    typename E::Frag a[KK][S::NF], bq[KK][S::NT];
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      const int ch = 4 * kk + (lane >> 4);
#pragma unroll
      for (int f = 0; f < S::NF; ++f) a[kk][f] = tile_row_frag<kQkvK>(st, hw * DH + 16 * f + (lane & 15), ch);
#pragma unroll
      for (int t = 0; t < S::NT; ++t)
        bq[kk][t] = tile_row_frag<kQkvK>(st, 2 * DH + S::TPW * tw + 16 * t + (lane & 15), ch);
    }
    issue(kb + kQkvStg - 1, nslot);
#pragma unroll
    for (int kk = 0; kk < KK; ++kk)
#pragma unroll
      for (int f = 0; f < S::NF; ++f)
#pragma unroll
        for (int t = 0; t < S::NT; ++t) acc[f][t] = E::mma(a[kk][f], bq[kk][t], acc[f][t]);
    slot = slot == kQkvStg - 1 ? 0 : slot + 1;
  }
  __builtin_amdgcn_s_waitcnt(0);  // the ring's last transfers land before the tile reuses the LDS
  __syncthreads();

  // product -> bf16 -> output tile [token][2 dh] (padded rows)
#pragma unroll
  for (int f = 0; f < S::NF; ++f)
#pragma unroll
    for (int t = 0; t < S::NT; ++t) {
      const int tok = S::TPW * tw + 16 * t + (lane & 15);
      const int col = hw * DH + 16 * f + 4 * (lane >> 4);
      uint2 v;
      v.x = uint32_t(f2bf(acc[f][t][0])) | (uint32_t(f2bf(acc[f][t][1])) << 16);
      v.y = uint32_t(f2bf(acc[f][t][2])) | (uint32_t(f2bf(acc[f][t][3])) << 16);
      *reinterpret_cast<uint2*>(smem + tok * S::OUTW + col) = v;
    }
  __syncthreads();

  if constexpr (GATE) {
    // output gate (relation.py:179-181): z = y * sigmoid(g) with g the bf16 product, the sigmoid
    // rounded to bf16 and the product rounded again, as the reference's bf16 ops round them; the
    // sigmoid is also written for the backward. The pair's 2 dh columns are contiguous (h1 = h0 + 1).
    constexpr int CH = 2 * DH / 8;
    for (int q = threadIdx.x; q < S::TOK * CH; q += 64 * NW) {
      const int tok = q / CH, c = q % CH;
      const int r = r0 + tok;
      if (r >= p.M) break;  // tasks go token by token: every later one is past M too
      const int64_t col = int64_t(h0) * DH + c * 8;
      const uint4 gv = *reinterpret_cast<const uint4*>(smem + tok * S::OUTW + c * 8);
      const uint4 yv = *reinterpret_cast<const uint4*>(p.gy + int64_t(r) * p.gy_sr + col);
      const uint32_t gw[4] = {gv.x, gv.y, gv.z, gv.w}, yw[4] = {yv.x, yv.y, yv.z, yv.w};
      uint32_t zw[4], sw[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const bf16_t s0 = f2bf(sigmoid_acc(bf2f(gw[k] & 0xffffu))), s1 = f2bf(sigmoid_acc(bf2f(gw[k] >> 16)));
        const bf16_t z0 = f2bf(bf2f(yw[k] & 0xffffu) * bf2f(s0)), z1 = f2bf(bf2f(yw[k] >> 16) * bf2f(s1));
        sw[k] = uint32_t(s0) | (uint32_t(s1) << 16);
        zw[k] = uint32_t(z0) | (uint32_t(z1) << 16);
      }
      *reinterpret_cast<uint4*>(p.gz + int64_t(r) * p.gz_sr + col) = make_uint4(zw[0], zw[1], zw[2], zw[3]);
      *reinterpret_cast<uint4*>(p.gs + int64_t(r) * p.gz_sr + col) = make_uint4(sw[0], sw[1], sw[2], sw[3]);
    }
    return;
  }

  if (part < 2 && p.nw1) {
    // QK-Norm of p1 / p2 before RoPE (relation.py:71-94, 208-210): per token and head, in fp32,
    // y = x rsqrt(mean(x^2) + eps) times the gain, rounded to bf16 in place in the tile (the
    // reference's HeadRMSNorm returns its input dtype); the pre-norm row is kept for the backward.
    const float* nw = part == 0 ? p.nw1 : p.nw2;
    for (int q = threadIdx.x; q < 2 * S::TOK; q += 64 * NW) {
      const int tok = q >> 1, hd = q & 1;
      bf16_t* row = smem + tok * S::OUTW + hd * DH;
      float ss = 0.f;
#pragma unroll
      for (int c = 0; c < DH / 8; ++c) {
        const uint4 v = *reinterpret_cast<const uint4*>(row + c * 8);
        const uint32_t vw[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const float a = bf2f(vw[k] & 0xffffu), b = bf2f(vw[k] >> 16);
          ss = fmaf(a, a, ss);
          ss = fmaf(b, b, ss);
        }
      }
      const float rr = rsqrtf(ss / float(DH) + p.eps);
      const int r = r0 + tok;
      const bool keep_raw = p.qkraw && r < p.M;
      const int bb = p.B == 1 ? 0 : r / p.T, tt = r - bb * p.T;
      bf16_t* raw = keep_raw ? p.qkraw + bb * p.qr_sb + int64_t(tt) * p.qr_sr + (part * p.H + (hd ? h1 : h0)) * DH
                             : nullptr;
#pragma unroll
      for (int c = 0; c < DH / 8; ++c) {
        const uint4 v = *reinterpret_cast<const uint4*>(row + c * 8);
        if (keep_raw) *reinterpret_cast<uint4*>(raw + c * 8) = v;
        const uint32_t vw[4] = {v.x, v.y, v.z, v.w};
        uint32_t ow[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const float a = (bf2f(vw[k] & 0xffffu) * rr) * nw[c * 8 + 2 * k];
          const float b = (bf2f(vw[k] >> 16) * rr) * nw[c * 8 + 2 * k + 1];
          ow[k] = uint32_t(f2bf(a)) | (uint32_t(f2bf(b)) << 16);
        }
        *reinterpret_cast<uint4*>(row + c * 8) = make_uint4(ow[0], ow[1], ow[2], ow[3]);
      }
    }
    __syncthreads();
  }

  // rotations and stores. The chunks of a token row pair up: RoPE pairs chunk cc of a head with
  // chunk cc + dh/16 of the same head (the two halves, one table entry for both), Givens pairs chunk
  // cc of the first head with chunk cc of the second. A task is one pair of one token row: two
  // chunks in, two rotated chunks out.
  const bool rope = part < 2 && p.tab != nullptr;
  const bool giv = part == 2 && p.theta != nullptr;
  float gc = 1.f, gs = 0.f;
  if (giv) {
    float sn, cs;
    sincosf(p.theta[hp], &sn, &cs);
    gc = bf2f(f2bf(cs));
    gs = bf2f(f2bf(sn));
  }
  constexpr int HC = DH / 16;  // chunks per half head
  constexpr int CPH = DH / 8;  // chunks per head
  constexpr int NPAIR = CPH;   // pairs per token row (2 heads x CPH chunks / 2)
  bf16_t* obase = part == 0 ? p.o1 : (part == 1 ? p.o2 : p.o3);
  const int64_t osb = part == 0 ? p.o1_sb : (part == 1 ? p.o2_sb : p.o3_sb);
  const int64_t osh = part == 0 ? p.o1_sh : (part == 1 ? p.o2_sh : p.o3_sh);
  const int64_t osr = part == 0 ? p.o1_sr : (part == 1 ? p.o2_sr : p.o3_sr);
  // every table load of the thread's tasks first (one latency for all of them), then the rotations
  constexpr int NTASK = S::TOK * NPAIR / (64 * NW);
  static_assert(S::TOK * NPAIR % (64 * NW) == 0, "whole tasks per thread");
  const int rlast = p.M - 1;
  uint4 tabv[NTASK][2];
  if (rope) {
#pragma unroll
    for (int i = 0; i < NTASK; ++i) {
      const int q = threadIdx.x + 64 * NW * i;
      const int tok = q / NPAIR, cc = (q % NPAIR) % HC;
      const int r = min(r0 + tok, rlast);
      const int t = p.B == 1 ? r : r % p.T;
      const uint4* tp = reinterpret_cast<const uint4*>(p.tab + int64_t(t) * (DH / 2) + cc * 8);
      tabv[i][0] = tp[0];
      tabv[i][1] = tp[1];
    }
  }
#pragma unroll
  for (int i = 0; i < NTASK; ++i) {
    const int q = threadIdx.x + 64 * NW * i;
    const int tok = q / NPAIR, j = q % NPAIR;
    const int r = r0 + tok;
    if (r >= p.M) break;  // tokens are in order: every later task of this thread is past M too
    const int b = p.B == 1 ? 0 : r / p.T, t = r - b * p.T;
    // chunk ca (head ha, chunk cca) and its partner cb (head hb, chunk ccb); out_a = x_a C - x_b S,
    // out_b = x_b C + x_a S
    int ha, cca, hb, ccb;
    if (part < 2) {
      ha = hb = j / HC;
      cca = j % HC;
      ccb = cca + HC;
    } else {
      ha = 0;
      hb = 1;
      cca = ccb = j;
    }
    const uint4 xa = *reinterpret_cast<const uint4*>(smem + tok * S::OUTW + (ha * CPH + cca) * 8);
    const uint4 xb = *reinterpret_cast<const uint4*>(smem + tok * S::OUTW + (hb * CPH + ccb) * 8);
    const int gha = ha ? h1 : h0, ghb = hb ? h1 : h0;
    if (part == 2 && p.iraw) {
      *reinterpret_cast<uint4*>(p.iraw + b * p.ir_sb + t * p.ir_sr + gha * DH + cca * 8) = xa;
      *reinterpret_cast<uint4*>(p.iraw + b * p.ir_sb + t * p.ir_sr + ghb * DH + ccb * 8) = xb;
    }
    float C[8], Sn[8];
    if (rope) {
      const uint32_t tv[8] = {tabv[i][0].x, tabv[i][0].y, tabv[i][0].z, tabv[i][0].w,
                              tabv[i][1].x, tabv[i][1].y, tabv[i][1].z, tabv[i][1].w};
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        C[e] = bf2f(tv[e] & 0xffffu);
        Sn[e] = bf2f(tv[e] >> 16);
      }
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        C[e] = gc;
        Sn[e] = gs;
      }
    }
    const uint32_t aw[4] = {xa.x, xa.y, xa.z, xa.w}, bw[4] = {xb.x, xb.y, xb.z, xb.w};
    uint32_t oa[4], ob[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const float a0 = bf2f(aw[k] & 0xffffu), a1 = bf2f(aw[k] >> 16);
      const float b0 = bf2f(bw[k] & 0xffffu), b1 = bf2f(bw[k] >> 16);
      const float c0 = C[2 * k], c1 = C[2 * k + 1], s0 = Sn[2 * k], s1 = Sn[2 * k + 1];
      oa[k] = uint32_t(f2bf(rot_round<bf16_t>(a0, c0, b0, -s0))) |
              (uint32_t(f2bf(rot_round<bf16_t>(a1, c1, b1, -s1))) << 16);
      ob[k] = uint32_t(f2bf(rot_round<bf16_t>(b0, c0, a0, s0))) |
              (uint32_t(f2bf(rot_round<bf16_t>(b1, c1, a1, s1))) << 16);
    }
    *reinterpret_cast<uint4*>(obase + b * osb + t * osr + gha * osh + cca * 8) = make_uint4(oa[0], oa[1], oa[2], oa[3]);
    *reinterpret_cast<uint4*>(obase + b * osb + t * osr + ghb * osh + ccb * 8) = make_uint4(ob[0], ob[1], ob[2], ob[3]);
  }
}

// ------------------------------------------------------------------------------------------------
// host side
// ------------------------------------------------------------------------------------------------
size_t qkv_rope_workspace_bytes(const mote_qkv_rope_args* a) {
  if (!a->inv_freq || a->T <= 0 || a->D <= 0) return 0;
  return size_t(a->T) * (a->D / 2) * sizeof(uint32_t);
}

// One launch of the kernel for head dim DH: token tiles of the workgroup size DH takes, whole rounds of
// the grid over the 8 XCDs (the extra ids return).
template <int DH, bool GATE>
static void launch_qkv_kernel(QkvParams p, int64_t M, hipStream_t stream) {
  constexpr int NW = qkv_waves<DH>();
  p.ntok = int((M + QkvShape<DH, NW>::TOK - 1) / QkvShape<DH, NW>::TOK);
  const int nwg = p.ntok * p.ncol;
  hipLaunchKernelGGL((qkv_rope_kernel<DH, NW, GATE>), dim3(unsigned((nwg + 7) / 8 * 8)), dim3(64 * NW), 0, stream, p);
}

static bool al16v(const void* ptr, int64_t s0, int64_t s1, int64_t s2) {
  return reinterpret_cast<uintptr_t>(ptr) % 16 == 0 && (s0 * 2) % 16 == 0 && (s1 * 2) % 16 == 0 &&
         (s2 * 2) % 16 == 0;
}

int launch_qkv_rope_fwd(const mote_qkv_rope_args* a, hipStream_t stream) {
  if (!a) return set_error(MOTE_ERR_ARGUMENT, "qkv_rope: null args");
  if (a->D != 64 && a->D != 96 && a->D != 128)
    return set_error(MOTE_ERR_SHAPE, "qkv_rope: head dim %d (the fused prologue serves 64, 96, 128)", a->D);
  if (a->B < 0 || a->T < 0 || a->H < 2 || a->H % 2)
    return set_error(MOTE_ERR_SHAPE, "qkv_rope: B = %d, T = %d, H = %d (H even)", a->B, a->T, a->H);
  const int K = a->H * a->D;
  if (K % kQkvK) return set_error(MOTE_ERR_SHAPE, "qkv_rope: model width %d not a multiple of 32", K);
  const int64_t M = int64_t(a->B) * a->T;
  if (M == 0) return MOTE_OK;
  if (M > (int64_t(1) << 30)) return set_error(MOTE_ERR_SHAPE, "qkv_rope: %lld tokens", (long long)M);
  if (!a->x || !a->w || !a->p1.data || !a->p2.data || !a->info.data)
    return set_error(MOTE_ERR_ARGUMENT, "qkv_rope: null pointer");
  if (a->B > 1 && a->x_sb != int64_t(a->T) * a->x_sr)
    return set_error(MOTE_ERR_ARGUMENT, "qkv_rope: x must hold its batches back to back (x_sb == T * x_sr)");
  if (a->x_sr >= (int64_t(1) << 23) || a->w_sr >= (int64_t(1) << 23))
    return set_error(MOTE_ERR_ARGUMENT, "qkv_rope: row strides must stay below 2^23 elements");
  if (!al16v(a->x, a->x_sr, 0, 0) || !al16v(a->w, a->w_sr, 0, 0) ||
      !al16v(a->p1.data, a->p1.stride_b, a->p1.stride_h, a->p1.stride_r) ||
      !al16v(a->p2.data, a->p2.stride_b, a->p2.stride_h, a->p2.stride_r) ||
      !al16v(a->info.data, a->info.stride_b, a->info.stride_h, a->info.stride_r) ||
      (a->info_raw && !al16v(a->info_raw, a->ir_sb, a->ir_sr, 0)) ||
      (a->qk_raw && !al16v(a->qk_raw, a->qr_sb, a->qr_sr, 0)))
    return set_error(MOTE_ERR_ARGUMENT, "qkv_rope: rows must start on 16-byte boundaries");
  if ((a->norm_w1 == nullptr) != (a->norm_w2 == nullptr) || (a->qk_raw && !a->norm_w1))
    return set_error(MOTE_ERR_ARGUMENT, "qkv_rope: QK-Norm needs both gains (and qk_raw only with them)");
  if (a->inv_freq && (!a->workspace || a->workspace_bytes < qkv_rope_workspace_bytes(a) ||
                      reinterpret_cast<uintptr_t>(a->workspace) % 16))
    return set_error(MOTE_ERR_WORKSPACE, "qkv_rope: workspace too small or misaligned");
  QkvParams p;
  p.x = reinterpret_cast<const bf16_t*>(a->x); p.x_sr = a->x_sr;
  p.w = reinterpret_cast<const bf16_t*>(a->w); p.w_sr = a->w_sr;
  p.tab = a->inv_freq ? reinterpret_cast<const uint32_t*>(a->workspace) : nullptr;
  p.theta = a->theta;
  p.o1 = reinterpret_cast<bf16_t*>(a->p1.data); p.o1_sb = a->p1.stride_b; p.o1_sh = a->p1.stride_h; p.o1_sr = a->p1.stride_r;
  p.o2 = reinterpret_cast<bf16_t*>(a->p2.data); p.o2_sb = a->p2.stride_b; p.o2_sh = a->p2.stride_h; p.o2_sr = a->p2.stride_r;
  p.o3 = reinterpret_cast<bf16_t*>(a->info.data); p.o3_sb = a->info.stride_b; p.o3_sh = a->info.stride_h;
  p.o3_sr = a->info.stride_r;
  p.iraw = reinterpret_cast<bf16_t*>(a->info_raw); p.ir_sb = a->ir_sb; p.ir_sr = a->ir_sr;
  p.nw1 = a->norm_w1; p.nw2 = a->norm_w2; p.eps = a->norm_eps;
  p.qkraw = reinterpret_cast<bf16_t*>(a->qk_raw); p.qr_sb = a->qr_sb; p.qr_sr = a->qr_sr;
  p.gy = nullptr; p.gy_sr = 0; p.gz = p.gs = nullptr; p.gz_sr = 0;
  p.B = a->B; p.T = a->T; p.H = a->H; p.K = K; p.M = int(M); p.parity = a->layer_parity & 1; p.nk = K / kQkvK;
  p.ncol = 3 * (a->H / 2);
  if (a->inv_freq && !a->table_ready) {
    const int64_t n = int64_t(a->T) * (a->D / 2);
    hipLaunchKernelGGL(rope_table_kernel, dim3(unsigned((n + 255) / 256)), dim3(256), 0, stream, a->inv_freq, a->pos0,
                       a->T, a->D / 2, reinterpret_cast<uint32_t*>(a->workspace));
    int rc = check_launch("qkv_rope/table");
    if (rc) return rc;
  }
  switch (a->D) {
    case 64: launch_qkv_kernel<64, false>(p, M, stream); break;
    case 96: launch_qkv_kernel<96, false>(p, M, stream); break;
    default: launch_qkv_kernel<128, false>(p, M, stream); break;
  }
  return check_launch("qkv_rope");
}

// The output gate's product on the same kernel: the D columns of x wg^T are tiled as D / (2 dh)
// "head pairs", dh the first of {64, 96, 128} that divides them up to 32,768 rows and of
// {96, 128, 64} beyond (the narrower tiles give more workgroups where the rows are few). At D 768:
// 16.3 / 19.8 / 27.0 / 47.7 us at 1,241 / 4,964 / 9,928 / 19,856 rows as dh 64 pairs against
// 22.2 / 25.9 / 31.8 / 51.5 as dh 96 pairs; 213 against 194 us at 79,424 rows; dh 128 pairs took
// 40 / 197 us at 4,964 / 79,424. Every output column's sum runs over k in the same order whatever
// the tiling, so the results do not depend on it.
int launch_gate_product(const mote_gate_product_args* a, hipStream_t stream) {
  if (!a) return set_error(MOTE_ERR_ARGUMENT, "gate_product: null args");
  if (a->B < 0 || a->T < 0 || a->D <= 0) return set_error(MOTE_ERR_SHAPE, "gate_product: bad sizes");
  int DH = 0;
  const bool few = int64_t(a->B) * a->T <= 32768;
  for (const int c : {few ? 64 : 96, few ? 96 : 128, few ? 128 : 64})
    if (a->D % (2 * c) == 0) { DH = c; break; }
  if (!DH || a->D % kQkvK) return set_error(MOTE_ERR_SHAPE, "gate_product: width %d (needs a multiple of 128)", a->D);
  const int64_t M = int64_t(a->B) * a->T;
  if (M == 0) return MOTE_OK;
  if (M > (int64_t(1) << 30)) return set_error(MOTE_ERR_SHAPE, "gate_product: %lld tokens", (long long)M);
  if (!a->x || !a->w || !a->y || !a->z || !a->s) return set_error(MOTE_ERR_ARGUMENT, "gate_product: null pointer");
  if (a->x_sr >= (int64_t(1) << 23) || a->w_sr >= (int64_t(1) << 23))
    return set_error(MOTE_ERR_ARGUMENT, "gate_product: row strides must stay below 2^23 elements");
  if (!al16v(a->x, a->x_sr, 0, 0) || !al16v(a->w, a->w_sr, 0, 0) || !al16v(a->y, a->y_sr, 0, 0) ||
      !al16v(a->z, a->z_sr, 0, 0) || !al16v(a->s, a->z_sr, 0, 0))
    return set_error(MOTE_ERR_ARGUMENT, "gate_product: rows must start on 16-byte boundaries");
  QkvParams p = {};
  p.x = reinterpret_cast<const bf16_t*>(a->x); p.x_sr = a->x_sr;
  p.w = reinterpret_cast<const bf16_t*>(a->w); p.w_sr = a->w_sr;
  p.gy = reinterpret_cast<const bf16_t*>(a->y); p.gy_sr = a->y_sr;
  p.gz = reinterpret_cast<bf16_t*>(a->z); p.gs = reinterpret_cast<bf16_t*>(a->s); p.gz_sr = a->z_sr;
  p.B = 1; p.T = int(M); p.H = a->D / DH; p.K = a->D; p.M = int(M); p.parity = 0; p.nk = a->D / kQkvK;
  p.ncol = p.H / 2;
  switch (DH) {
    case 64: launch_qkv_kernel<64, true>(p, M, stream); break;
    case 96: launch_qkv_kernel<96, true>(p, M, stream); break;
    default: launch_qkv_kernel<128, true>(p, M, stream); break;
  }
  return check_launch("gate_product");
}

}  // namespace mote
