// Skinny product for the decode engine's projections: y [B, N] = x [B, K] W[N, K]^T in bf16 with
// fp32 accumulation, B <= 16 (one new chunk per sequence), the shape of the per-token projections
// around the Relation decode step (the stacked [w1; w2; wi] before it and wo after it,
// mote/infer/graph.py:151-187). At these shapes the work is reading W once (3.5 MB for the stacked
// Mote-96M projection), so the kernel is laid out for bandwidth and latency, not for reuse:
//
//   one workgroup (4 waves) per 16 rows of W; wave w takes the k range [w K/4, (w+1) K/4) and runs
//   C[16 features][16 batch] += W_strip x^T on v_mfma_f32_16x16x32_bf16, with every 16-byte load of
//   its W rows and x rows issued before the first product (A fragment: lane (r = l % 16, q = l / 16)
//   holds W[n0 + r][k + 8q .. +8], 64-byte runs per row; B fragment: x[b = l % 16][k + 8q .. +8],
//   zero for b >= B); the four partial tiles add through LDS in a fixed order and wave 0 rounds and
//   stores y[b][n0 + r] for b < B. Optionally workgroup 0 also writes the decode step's exchange mass
//   xm[b], the mean of g[b] over the heads (the decode launch then needs no count of its finished
//   heads for it).
#include "common.hpp"
#include "params.hpp"

namespace mote {

constexpr int kSkWaves = 4;
constexpr int kSkMaxKs = 8;  // 32-wide k steps per wave held in registers: K <= 4 * 8 * 32 = 1024

struct SkinnyParams {
  const bf16_t* x; int64_t x_sr;
  const bf16_t* w; int64_t w_sr;
  bf16_t* y; int64_t y_sr;
  const unsigned char* run;  // predicate: 0 -> the launch writes nothing (null: always run)
  const float* g; float* xm;  // optional: xm[b] = mean of g[b][0 .. heads) (the decode step's exchange mass)
  int B, N, K, heads;
};

template <int KS>
__global__ void __launch_bounds__(64 * kSkWaves) skinny_gemm_kernel(const SkinnyParams p) {
  using E = Elem<bf16_t>;
  using Frag = E::Frag;
  __shared__ __align__(16) float part[kSkWaves][16][17];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, q = lane >> 4;
  const int n0 = blockIdx.x * 16;
  const int kw = p.K / kSkWaves;  // a multiple of 32 (host check)
  const int k0 = wave * kw;
  const int nks = kw / 32;        // <= KS
  const bf16_t* wrow = p.w + int64_t(n0 + r) * p.w_sr + k0 + 8 * q;
  const bool has_b = r < p.B;
  const bf16_t* xrow = p.x + int64_t(has_b ? r : 0) * p.x_sr + k0 + 8 * q;
  Frag a[KS], bx[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s) {
    if (s < nks) {
      a[s] = E::load8(wrow + 32 * s);
      bx[s] = E::load8(xrow + 32 * s);
    }
  }
  // the decode step's exchange mass (graph.py:186) on the side: workgroup 0, wave 1, lane b < B
  // sums g[b][0 .. heads) in head order
  const int xb = int(threadIdx.x) - 64;
  const bool xm_lane = p.xm != nullptr && blockIdx.x == 0 && xb >= 0 && xb < p.B;
  float gsum = 0.f;
  if (xm_lane)
    for (int h = 0; h < p.heads; ++h) gsum += p.g[int64_t(xb) * p.heads + h];
  // the predicate after the loads are issued (reads are harmless); uniform, so the whole
  // workgroup leaves before its barrier
  if (p.run && p.run[0] == 0) return;
  if (xm_lane) p.xm[xb] = gsum / float(p.heads);
  f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < KS; ++s) {
    if (s < nks) {
      const Frag b = has_b ? bx[s] : E::zero();
      acc = E::mma(a[s], b, acc);
    }
  }
  // C[feature 4 q + i][batch r] of this wave's k range
#pragma unroll
  for (int i = 0; i < 4; ++i) part[wave][4 * q + i][r] = acc[i];
  __syncthreads();
  if (wave == 0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int f = 4 * q + i;
      float v = part[0][f][r];
#pragma unroll
      for (int w = 1; w < kSkWaves; ++w) v += part[w][f][r];
      if (has_b) p.y[int64_t(r) * p.y_sr + n0 + f] = E::from_f(v);
    }
  }
}

int launch_skinny_gemm(const mote_skinny_gemm_args* a, hipStream_t stream) {
  if (!a) return set_error(MOTE_ERR_ARGUMENT, "skinny_gemm: null args");
  if (a->dtype != MOTE_BF16) return set_error(MOTE_ERR_ARGUMENT, "skinny_gemm: bf16 only (dtype %d)", a->dtype);
  if (a->B < 0 || a->B > 16) return set_error(MOTE_ERR_SHAPE, "skinny_gemm: B = %d (at most 16 rows)", a->B);
  if (a->N <= 0 || a->N % 16 || a->K <= 0 || a->K % (32 * kSkWaves) || a->K > 32 * kSkWaves * kSkMaxKs)
    return set_error(MOTE_ERR_SHAPE, "skinny_gemm: N = %d (a multiple of 16), K = %d (a multiple of 128, at most %d)",
                     a->N, a->K, 32 * kSkWaves * kSkMaxKs);
  if (a->B == 0) return MOTE_OK;
  if (!a->x || !a->w || !a->y) return set_error(MOTE_ERR_ARGUMENT, "skinny_gemm: null pointer");
  if (a->xm && (!a->g || a->heads <= 0))
    return set_error(MOTE_ERR_ARGUMENT, "skinny_gemm: xm needs g and heads > 0");
  if (reinterpret_cast<uintptr_t>(a->x) % 16 || reinterpret_cast<uintptr_t>(a->w) % 16 || (a->x_sr * 2) % 16 ||
      (a->w_sr * 2) % 16 || reinterpret_cast<uintptr_t>(a->y) % 2)
    return set_error(MOTE_ERR_ARGUMENT, "skinny_gemm: x and W rows must start on 16-byte boundaries");
  if (a->x_sr < a->K || a->w_sr < a->K || (a->B > 1 && a->y_sr < a->N))
    return set_error(MOTE_ERR_ARGUMENT, "skinny_gemm: row strides shorter than the rows");
  SkinnyParams p;
  p.x = reinterpret_cast<const bf16_t*>(a->x); p.x_sr = a->x_sr;
  p.w = reinterpret_cast<const bf16_t*>(a->w); p.w_sr = a->w_sr;
  p.y = reinterpret_cast<bf16_t*>(a->y); p.y_sr = a->y_sr;
  p.run = a->run;
  p.g = a->xm ? a->g : nullptr; p.xm = a->xm; p.heads = a->xm ? a->heads : 0;
  p.B = a->B; p.N = a->N; p.K = a->K;
  const int nks = a->K / (32 * kSkWaves);
  const dim3 grid(unsigned(a->N / 16)), block(64 * kSkWaves);
  if (nks <= 2) hipLaunchKernelGGL(skinny_gemm_kernel<2>, grid, block, 0, stream, p);
  else if (nks <= 4) hipLaunchKernelGGL(skinny_gemm_kernel<4>, grid, block, 0, stream, p);
  else hipLaunchKernelGGL(skinny_gemm_kernel<kSkMaxKs>, grid, block, 0, stream, p);
  return check_launch("skinny_gemm");
}

}  // namespace mote
