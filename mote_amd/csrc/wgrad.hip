// Weight gradient of a projection: dW [N, K] = A^T X for A [M, N] (the output gradient, token rows)
// and X [M, K] (the projection's input rows), bf16 in and out, fp32 accumulation. This is the
// weight half of autograd through the projections of FullRelation (mote/model/relation.py:204-215:
// the stacked [w1; w2; wi] product, whose weight gradient is dqkv^T x), the product whose reduction
// runs over the M token rows.
//
// A workgroup (4 waves) owns a 128 x 128 tile of dW and one contiguous range of token rows (a split
// of M); the k of the products is the token index. Stages of 64 token rows of both operands go
// global -> LDS by direct transfers into two slots ([token][128 columns], chunks swizzled as in
// tiles.hpp), and both MFMA operands are transposed LDS reads (ds_read_b64_tr_b16) of the staged
// tiles, so neither operand is transposed in memory. Wave (wr, wc) holds dW rows 64 wr .. +63 and
// columns 64 wc .. +63 as 4 x 4 accumulator tiles with the X columns in the accumulator rows, so a
// lane ends with 4 consecutive columns of one dW row (one 8-byte bf16 store).
//
// Splits: with few dW tiles (2304 x 768 is 108 of them) M is cut into S ranges of whole 64-row
// stages, S about two workgroups per CU over the tiles; each split writes its fp32 partial tile to
// the workspace and a second launch adds the S partials in split order and rounds once to bf16
// (bitwise reproducible, independent of scheduling). One split writes bf16 directly. Rows past M in
// the last stage are zeroed in LDS in both operands.
#include "common.hpp"
#include "params.hpp"
#include "tiles.hpp"

namespace mote {

int device_cu_count();

constexpr int kWgTok = 64;    // token rows per stage (two 32-deep k steps)
constexpr int kWgTile = 128;  // rows and columns of dW per workgroup
constexpr int kWgWaves = 4;

struct WgradParams {
  const bf16_t* a; int64_t a_sr;  // [M, N]
  const bf16_t* x; int64_t x_sr;  // [M, K]
  bf16_t* dw; int64_t dw_sr;      // [N, K]
  float* part;                    // [nsplit][N][K] fp32 partials, or null (one split: bf16 straight to dw)
  int M, N, K, nsplit, mper, ntn, ntk;
};

__global__ void __launch_bounds__(64 * kWgWaves) __attribute__((amdgpu_waves_per_eu(2)))
wgrad_kernel(const WgradParams p) {
  using E = Elem<bf16_t>;
  using Frag = E::Frag;
  using St = TileStager<kWgTile, kWgWaves, 2>;
  constexpr int TILE = kWgTok * kWgTile;  // elements of one staged operand tile
  constexpr int STAGE = 2 * TILE;         // X tile | A tile
  __shared__ __align__(16) bf16_t smem[2 * STAGE];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int li = lane & 15, lg = lane >> 4;
  // workgroup id -> (split, row tile, column tile): workgroups go round-robin over the 8 XCDs, so XCD
  // j takes the j-th contiguous run of that order, tiles of one split that share their operand rows
  const int per_split = p.ntn * p.ntk, nwg = per_split * p.nsplit, per = (nwg + 7) / 8;
  const int seq = (blockIdx.x % 8) * per + blockIdx.x / 8;
  if (seq >= nwg) return;
  const int split = seq / per_split, rem = seq - split * per_split;
  const int tn = rem / p.ntk, tk = rem - tn * p.ntk;
  const int m0 = split * p.mper, m1 = min(p.M, m0 + p.mper);
  const int nblk = (m1 - m0 + kWgTok - 1) / kWgTok;
  const bf16_t* const src[2] = {p.x + int64_t(tk) * kWgTile, p.a + int64_t(tn) * kWgTile};
  const int64_t stride[2] = {p.x_sr, p.a_sr};
  St st;
  st.init(wave, lane, stride);
  const int wr = wave & 1, wc = wave >> 1;

  f32x4 acc[4][4];  // [X column tile i][A column tile j]
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  st.issue(smem, src, stride, m0, p.M - 1, wave, lane);
  for (int b = 0; b < nblk; ++b) {
    bf16_t* cur = smem + (b & 1) * STAGE;
    __builtin_amdgcn_s_waitcnt(0);  // this wave's transfers of stage b
    lds_barrier();
    const int r0 = m0 + b * kWgTok;
    if (r0 + kWgTok > p.M) {
      // the last stage of the reduction: its rows past M hold copies of row M - 1; zero them in both
      // tiles (whole rows, so the chunk swizzle does not matter)
      const int nz = r0 + kWgTok - p.M;
      for (int q = threadIdx.x; q < 2 * nz * (kWgTile / 8); q += 64 * kWgWaves) {
        const int t = q / (nz * (kWgTile / 8)), w = q - t * (nz * (kWgTile / 8));
        const int row = p.M - r0 + w / (kWgTile / 8), ch = w % (kWgTile / 8);
        *reinterpret_cast<bf16x8*>(cur + t * TILE + row * kWgTile + ch * 8) = bf16x8{};
      }
      lds_barrier();
    }
    // every fragment of the stage, then the next stage's transfers into the other slot, then the
    // products (the other slot's last reads were the previous stage's, before this barrier)
    Frag fx[2][4], fa[2][4];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        fx[ks][i] = tile_tr_frag<kWgTile>(cur, 32 * ks, 4 * wc + i, li, lg);
        fa[ks][i] = tile_tr_frag<kWgTile>(cur + TILE, 32 * ks, 4 * wr + i, li, lg);
      }
    if (b + 1 < nblk) st.issue(smem + ((b + 1) & 1) * STAGE, src, stride, r0 + kWgTok, p.M - 1, wave, lane);
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = E::mma(fx[ks][i], fa[ks][j], acc[i][j]);
  }

  // lane: dW row n = 128 tn + 64 wr + 16 j + li, columns c = 128 tk + 64 wc + 16 i + 4 lg .. +3
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int n = tn * kWgTile + 64 * wr + 16 * j + li;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = tk * kWgTile + 64 * wc + 16 * i + 4 * lg;
      if (p.part) {
        float* dst = p.part + (int64_t(split) * p.N + n) * p.K + c;
        *reinterpret_cast<float4*>(dst) = make_float4(acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]);
      } else {
        uint2 v;
        v.x = uint32_t(f2bf(acc[i][j][0])) | (uint32_t(f2bf(acc[i][j][1])) << 16);
        v.y = uint32_t(f2bf(acc[i][j][2])) | (uint32_t(f2bf(acc[i][j][3])) << 16);
        *reinterpret_cast<uint2*>(p.dw + int64_t(n) * p.dw_sr + c) = v;
      }
    }
  }
}

// dW = the sum of the splits' partials in split order, rounded once; no splits (M = 0): zeros.
// Four consecutive columns per thread.
__global__ void __launch_bounds__(256) wgrad_sum_kernel(const WgradParams p) {
  const int64_t q = int64_t(blockIdx.x) * 256 + threadIdx.x;
  const int64_t nq = int64_t(p.N) * (p.K / 4);
  if (q >= nq) return;
  const int n = int(q / (p.K / 4)), c = int(q % (p.K / 4)) * 4;
  float4 s = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int k = 0; k < p.nsplit; ++k) {
    const float4 v = *reinterpret_cast<const float4*>(p.part + (int64_t(k) * p.N + n) * p.K + c);
    s.x += v.x; s.y += v.y; s.z += v.z; s.w += v.w;
  }
  uint2 o;
  o.x = uint32_t(f2bf(s.x)) | (uint32_t(f2bf(s.y)) << 16);
  o.y = uint32_t(f2bf(s.z)) | (uint32_t(f2bf(s.w)) << 16);
  *reinterpret_cast<uint2*>(p.dw + int64_t(n) * p.dw_sr + c) = o;
}

// Splits of M: about two workgroups per CU over the dW tiles, at least four stages (256 rows) per
// split, every split a whole number of stages and none empty. Sets *mper (rows per split).
static int wgrad_splits(const mote_wgrad_args* a, int* mper) {
  const int tiles = (a->N / kWgTile) * (a->K / kWgTile);
  const int blocks = (a->M + kWgTok - 1) / kWgTok;
  int s = (2 * device_cu_count()) / (tiles > 0 ? tiles : 1);
  s = s < 1 ? 1 : s;
  const int cap = blocks / 4 < 1 ? 1 : blocks / 4;
  s = s < cap ? s : cap;
  const int per = (blocks + s - 1) / s;
  if (mper) *mper = per * kWgTok;
  return per > 0 ? (blocks + per - 1) / per : 1;
}

size_t wgrad_workspace_bytes(const mote_wgrad_args* a) {
  if (!a || a->M <= 0 || a->N <= 0 || a->K <= 0) return 0;
  const int s = wgrad_splits(a, nullptr);
  return s > 1 ? size_t(s) * size_t(a->N) * size_t(a->K) * sizeof(float) : 0;
}

int launch_wgrad(const mote_wgrad_args* a, hipStream_t stream) {
  if (!a) return set_error(MOTE_ERR_ARGUMENT, "wgrad: null args");
  if (a->dtype != MOTE_BF16) return set_error(MOTE_ERR_ARGUMENT, "wgrad: dtype %d (bf16 only)", a->dtype);
  if (a->M < 0 || a->N <= 0 || a->K <= 0 || a->N % kWgTile || a->K % kWgTile)
    return set_error(MOTE_ERR_SHAPE, "wgrad: M = %d, N = %d, K = %d (N and K multiples of 128)", a->M, a->N, a->K);
  if (!a->dw || (a->M > 0 && (!a->a || !a->x))) return set_error(MOTE_ERR_ARGUMENT, "wgrad: null pointer");
  if (a->a_sr < a->N || a->x_sr < a->K || a->dw_sr < a->K || a->a_sr >= (int64_t(1) << 24) ||
      a->x_sr >= (int64_t(1) << 24) || a->dw_sr >= (int64_t(1) << 40))
    return set_error(MOTE_ERR_ARGUMENT, "wgrad: row strides (a_sr >= N, x_sr >= K, dw_sr >= K; below 2^24 elements)");
  auto al16 = [](const void* ptr, int64_t sr) { return reinterpret_cast<uintptr_t>(ptr) % 16 == 0 && (sr * 2) % 16 == 0; };
  if ((a->M > 0 && (!al16(a->a, a->a_sr) || !al16(a->x, a->x_sr))) || !al16(a->dw, a->dw_sr))
    return set_error(MOTE_ERR_ARGUMENT, "wgrad: rows must start on 16-byte boundaries");
  WgradParams p;
  p.a = reinterpret_cast<const bf16_t*>(a->a); p.a_sr = a->a_sr;
  p.x = reinterpret_cast<const bf16_t*>(a->x); p.x_sr = a->x_sr;
  p.dw = reinterpret_cast<bf16_t*>(a->dw); p.dw_sr = a->dw_sr;
  p.M = a->M; p.N = a->N; p.K = a->K;
  p.ntn = a->N / kWgTile; p.ntk = a->K / kWgTile;
  p.part = nullptr;
  const int64_t nq = int64_t(a->N) * (a->K / 4);
  if (a->M == 0) {  // an empty reduction: dW = 0
    p.nsplit = 0; p.mper = 0;
    hipLaunchKernelGGL(wgrad_sum_kernel, dim3(unsigned((nq + 255) / 256)), dim3(256), 0, stream, p);
    return check_launch("wgrad/zero");
  }
  p.nsplit = wgrad_splits(a, &p.mper);
  if (p.nsplit > 1) {
    const size_t need = wgrad_workspace_bytes(a);
    if (!a->workspace || a->workspace_bytes < need || reinterpret_cast<uintptr_t>(a->workspace) % 16)
      return set_error(MOTE_ERR_WORKSPACE, "wgrad: workspace too small or misaligned (%zu bytes needed)", need);
    p.part = reinterpret_cast<float*>(a->workspace);
  }
  const int nwg = p.ntn * p.ntk * p.nsplit;
  hipLaunchKernelGGL(wgrad_kernel, dim3(unsigned((nwg + 7) / 8 * 8)), dim3(64 * kWgWaves), 0, stream, p);
  int rc = check_launch("wgrad");
  if (rc || p.nsplit == 1) return rc;
  hipLaunchKernelGGL(wgrad_sum_kernel, dim3(unsigned((nq + 255) / 256)), dim3(256), 0, stream, p);
  return check_launch("wgrad/sum");
}

}  // namespace mote
